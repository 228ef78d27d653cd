"""Convert the reference's MAC test vectors into a compact fixture.

The vectors are data files of the reference's own RTL testbench
(hardware/BQ/MAC_WXAY/testcase/w4a{4..8}/, read by tb_WXAY.sv:96-110): per case
(format kind nv = E5M3 block scale, mx = 5-bit power-of-two scale; weight width
4 bits = E2M1; activation width Y = 4..8 bits = E2M(Y-3); block size B) there are
4096 activation and 4096 weight codes, one scale byte per block and operand, the
fixed-point block dot product (psum), its fp16 scaled value and the fp16
accumulated output.  Nothing is executed: the text files are parsed as binary
numbers.  Block sizes 16, 32 and 128 are kept (the NVFP, MXFP and HBQ block sizes).

Usage:  python tests/golden/gen_rtl_kat.py [/root/reference]
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def read(path):
    with open(path) as f:
        return [l.strip() for l in f if l.strip()]


def main(ref="/root/reference"):
    base = os.path.join(ref, "hardware/BQ/MAC_WXAY/testcase")
    out = {}
    X = 4
    for Y in range(4, 9):
        for kind in ("nv", "mx"):
            for B in (16, 32, 128):
                stem = os.path.join(base, f"w{X}a{Y}", f"{kind}_w{X}a{Y}b{B}")
                key = f"{kind}_a{Y}_b{B}"
                ps = read(stem + "_psum.txt")
                width = len(ps[0])
                psum = np.array([int(v, 2) - ((int(v, 2) >> (width - 1)) << width) for v in ps], np.int32)
                out[key + "_act"] = np.array([int(v, 2) for v in read(stem + "_lp_act.txt")], np.uint8)
                out[key + "_wgt"] = np.array([int(v, 2) for v in read(stem + "_lp_wgt.txt")], np.uint8)
                out[key + "_scale_act"] = np.array([int(v, 2) for v in read(stem + "_scale_act.txt")], np.uint8)
                out[key + "_scale_wgt"] = np.array([int(v, 2) for v in read(stem + "_scale_wgt.txt")], np.uint8)
                out[key + "_psum"] = psum
                out[key + "_scaled_psum"] = np.array([int(v, 2) for v in read(stem + "_scaled_psum.txt")], np.uint16)
    np.savez_compressed(os.path.join(HERE, "rtl_mac_kat.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main(*sys.argv[1:])
