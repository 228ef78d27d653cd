"""CPU restatement of the packed HBQ wire format (numpy).

TEST INFRASTRUCTURE ONLY: tests/ use it as the checker of hbq_hbq_pack /
hbq_hbq_unpack; the product package ``hbq_amd`` never imports it.

Format (per row of a [rows, cols] tensor, blocks along the last dim):
  codes   cols fields of mbit + 3 bits: sign | 2-bit exponent field | mbit mantissa
          bits (exponent field 0 = subnormal), element i at bits [(mbit+3) i,
          (mbit+3)(i+1)) of the little-endian bit string.  This is the element
          order of LP_DATA (hardware/HBQ_accelerator/hbq_e_quantizer/top.sv:40-45)
          and of the MAC test vectors (hardware/BQ/MAC_WXAY/tb_WXAY.sv:174-180).
  l1      one E5M3 byte per block, exponent bias 15 (top.sv:23-26): bits [14:7] of
          the scale as fp16; 0xFF = not a finite E5M3 value.
  l2      l2_sc_bit bits per sub-block, LSB first (L2_SCALE, top.sv:44).
  scheme  one bit per block, LSB first (Mix only).
The decode is the reference's dequantization d = R(R(q l2[j][s]) l1)
(src/quantizer.py:790-796) from the level q of each code.
"""
import numpy as np

from . import oracle as O


# ---- element codes ---------------------------------------------------------------------

def level_of(mag, mbit):
    """E2Mm level (exponent field << mbit | mantissa) of a non-negative grid value."""
    mag = np.asarray(mag, np.float64)
    lev = np.zeros(mag.shape, np.int64)
    sub = mag < 1.0
    lev[sub] = np.round(mag[sub] * (1 << mbit)).astype(np.int64)
    e = np.floor(np.log2(np.where(sub, 1.0, mag))).astype(np.int64) + 1
    m = np.round((np.where(sub, 1.0, mag) / np.exp2(e - 1) - 1.0) * (1 << mbit)).astype(np.int64)
    lev[~sub] = (e[~sub] << mbit) | m[~sub]
    return lev


def level_value(level, mbit):
    """Magnitude of an E2Mm level."""
    level = np.asarray(level, np.int64)
    e, m = level >> mbit, level & ((1 << mbit) - 1)
    frac = m / float(1 << mbit)
    return np.where(e == 0, frac, (1.0 + frac) * np.exp2(np.maximum(e, 1) - 1))


def code_int(code, mbit):
    """Signed value of a code in units of 2^-mbit (an exact integer), as the MAC's
    fixed-point product path reads it (hardware/BQ/params.vh FIXED_SCALE)."""
    code = np.asarray(code, np.int64)
    w = mbit + 3
    s = (code >> (w - 1)) & 1
    e = (code >> mbit) & 3
    m = code & ((1 << mbit) - 1)
    a = np.where(e == 0, m, ((1 << mbit) + m) << np.maximum(e - 1, 0))
    return np.where(s == 1, -a, a)


# ---- E5M3 scale byte ---------------------------------------------------------------------

def e5m3_value(byte):
    b = np.asarray(byte, np.int64)
    e, m = b >> 3, b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -14, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 15))
    return np.where(e == 31, np.nan, v)


def e5m3_byte(v):
    v = np.asarray(v, np.float64)
    out = np.full(v.shape, 0xFF, np.int64)
    out[(v == 0) & ~np.signbit(v)] = 0
    ok = np.isfinite(v) & (v > 0) & (v <= 61440.0)
    sub = ok & (v < 2.0 ** -14)
    ms = v * 2.0 ** 17
    good_sub = sub & (ms == np.floor(ms)) & (ms < 8)
    out[good_sub] = ms[good_sub].astype(np.int64)
    nor = ok & ~sub
    e = np.floor(np.log2(np.where(nor, v, 1.0))).astype(np.int64)
    m8 = (np.where(nor, v, 1.0) / np.exp2(e) - 1.0) * 8.0
    good = nor & (m8 == np.floor(m8))
    out[good] = ((e[good] + 15) << 3) | m8[good].astype(np.int64)
    return out.astype(np.uint8)


# ---- T rounding of exact float64 values ------------------------------------------------------

def round_bits(v, dt):
    """RNE of float64 values (exact products here) to dt's bit patterns."""
    v = np.asarray(v, np.float64)
    if dt == "f16":
        with np.errstate(over="ignore"):          # overflow to inf is the rounding's result
            return v.astype(np.float16).view(np.uint16)
    f = v.astype(np.float32)                     # exact for the products decoded here
    if dt == "f32":
        return f
    b = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), b)


def bits_value(b, dt):
    b = np.asarray(b)
    if dt == "f16":
        return b.astype(np.uint16).view(np.float16).astype(np.float64)
    if dt == "bf16":
        return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return b.astype(np.float32).astype(np.float64)


# ---- codes of a reference quantization ------------------------------------------------------------

def hbq_codes(x, dt, res, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme, use_quant_kernel=True):
    """Element codes of HBQQuantizer.q's selected candidate (src/quantizer.py:781-791):
    t = R(x / l1_s), u = R(t / l2[j][s]), q = lpfp(u); code = sign | level(|q|).
    res is oracle.hbq_qdq's result for the same x and the same use_quant_kernel (the
    element rounding); the sign is that of its output."""
    x = O._bits(x, dt)
    rows, cols = x.shape
    tab = O.l2_table(l2_scheme, l2_sc_bit, dt).astype(np.float64)
    blk = np.arange(cols) // block_size
    sub = (np.arange(cols) % block_size) // l2_block_size
    s = res["scheme"][:, blk].astype(np.int64) if tab.shape[1] == 2 else np.zeros((rows, cols), np.int64)
    j = res["l2idx"][:, blk, sub].astype(np.int64)
    l1 = bits_value(res["l1"], dt)[:, blk]
    xv = bits_value(x, dt)
    t = bits_value(round_bits(xv / l1, dt), dt)
    u = round_bits(t / tab[j, s], dt)
    q = bits_value(O.elem_quant(u, dt, 2, mbit, compiled=use_quant_kernel), dt)
    lev = level_of(np.abs(q), mbit)
    y = res["y"]
    neg = np.signbit(y) if dt == "f32" else (y.astype(np.int64) >> 15) & 1
    return (lev | (neg.astype(np.int64) << (mbit + 2))).astype(np.uint8)


# ---- pack / unpack ---------------------------------------------------------------------------

def _bitstring(fields, w, nbytes):
    """LSB-first packing of rows of w-bit fields into nbytes per row."""
    rows, n = fields.shape
    bits = ((fields[:, :, None].astype(np.int64) >> np.arange(w)) & 1).reshape(rows, n * w)
    pad = nbytes * 8 - n * w
    bits = np.concatenate([bits, np.zeros((rows, pad), np.int64)], axis=1)
    return (bits.reshape(rows, nbytes, 8) << np.arange(8)).sum(-1).astype(np.uint8)


def _fields(bytes_, w, n):
    rows = bytes_.shape[0]
    bits = ((bytes_[:, :, None].astype(np.int64) >> np.arange(8)) & 1).reshape(rows, -1)[:, : n * w]
    return (bits.reshape(rows, n, w) << np.arange(w)).sum(-1)


def strides(cols, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme):
    nblk = cols // block_size
    return (cols * (mbit + 3) // 8, nblk, (cols // l2_block_size * l2_sc_bit + 7) // 8,
            (nblk + 7) // 8 if l2_scheme == "Mix" else 0)


def pack(codes, l1, l2idx, scheme, dt, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme):
    """codes [rows, cols] (one per element), l1 [rows, nblk] dt bits, l2idx [rows, nblk, nsub],
    scheme [rows, nblk] -> dict of the four byte strings."""
    codes = np.asarray(codes, np.int64)
    rows, cols = codes.shape
    st = strides(cols, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme)
    out = {"codes": _bitstring(codes & ((1 << (mbit + 3)) - 1), mbit + 3, st[0]),
           "l1": e5m3_byte(bits_value(l1, dt)),
           "l2": _bitstring(np.asarray(l2idx, np.int64).reshape(rows, -1), l2_sc_bit, st[2]) if l2_sc_bit else None,
           "scheme": _bitstring(np.asarray(scheme, np.int64), 1, st[3]) if l2_scheme == "Mix" else None}
    return out


def unpack(p, rows, cols, dt, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme):
    """The four byte strings -> y [rows, cols] in dt bits: R(R(level l2[j][s]) l1) with the sign."""
    w = mbit + 3
    code = _fields(p["codes"], w, cols)
    tab = O.l2_table(l2_scheme, l2_sc_bit, dt).astype(np.float64)
    blk = np.arange(cols) // block_size
    nblk = cols // block_size
    s = _fields(p["scheme"], 1, nblk)[:, blk] if l2_scheme == "Mix" else np.zeros((rows, cols), np.int64)
    j = _fields(p["l2"], l2_sc_bit, cols // l2_block_size)[:, np.arange(cols) // l2_block_size] if l2_sc_bit \
        else np.zeros((rows, cols), np.int64)
    l1 = e5m3_value(p["l1"])[:, blk]
    mag = level_value(code & ((1 << (mbit + 2)) - 1), mbit)
    a = bits_value(round_bits(mag * tab[j, s], dt), dt)
    d = bits_value(round_bits(a * l1, dt), dt)
    d = np.where((code >> (mbit + 2)) & 1 == 1, -d, d)
    return round_bits(d, dt)
