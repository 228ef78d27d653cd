// One HBQ block (HBQQuantizer.q for one block, src/quantizer.py:741-859) held
// by lpb lanes of 16 elements each: the direct evaluation of every L2
// candidate of every scheme, in T's rounding, with the sub-block and block
// errors summed in torch's order.  Used by the generic kernel and as the exact
// fallback of the table-driven kernels.
#pragma once
#include "hbq_numeric.h"
#include "quant_common.h"

namespace hbq {

// xv: this lane's 16 elements; li: lane within the block; lane: lane in the wave.
// Outputs: out (dequantized), cout (codes), l1sel (L1 scale of the chosen
// scheme), sstar (chosen scheme), jsel (chosen L2 candidate of each of this
// lane's sub-blocks, for the chosen scheme).
template <class T, int M, int L2B, int S>
__device__ __forceinline__ void hbq_block(const float* xv, int li, int lpb, int lane, const HbqParams& p, float* out,
                                          uint32_t* cout, float& l1sel, int& sstar, int* jsel_out) {
    constexpr int NSUBL = L2B <= kV ? kV / L2B : 1;   // sub-blocks held by one lane
    constexpr int LPS = L2B <= kV ? 1 : L2B / kV;     // lanes per sub-block
    const int lane_base = lane - li;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        uint32_t b = f2bits(xv[i]) & 0x7fffffffu;
        m = m > b ? m : b;
    }
    const float amax = bits2f(group_max_bits(m, lpb));

    float l1[S];
    float dsel[S][kV], sqsel[S][kV];
    uint32_t csel[S][kV];
    int jsel[S][NSUBL];

#pragma unroll
    for (int s = 0; s < S; ++s) {
        l1[s] = scale_quant<T>(T::round(amax / p.em[s]), p.sf);
        const float rl1 = 1.0f / l1[s];
        float t[kV];
#pragma unroll
        for (int i = 0; i < kV; ++i) t[i] = div_T<T>(xv[i], l1[s], rl1);
        float best[NSUBL];
        for (int j = 0; j < p.J; ++j) {
            const float l2 = p.l2[j][s], rl2 = p.rl2[j][s];
            float dj[kV], sqj[kV];
            uint32_t cj[kV];
#pragma unroll
            for (int i = 0; i < kV; ++i) {
                float u = (l2 == 1.0f) ? t[i] : div_T<T>(t[i], l2, rl2);
                float q = elem_quant<T, M>(u, cj[i], p.fused);
                float d = T::round(T::round(q * l2) * l1[s]);
                float e = T::round(xv[i] - d);
                dj[i] = d;
                sqj[i] = T::round(e * e);
            }
#pragma unroll
            for (int sb = 0; sb < NSUBL; ++sb) {
                constexpr int n = L2B <= kV ? L2B : kV;
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < n; ++i) acc += sqj[sb * n + i];
                if constexpr (LPS == 2) {
                    // a lane pair: DPP swap within the pair (quad_perm 1,0,3,2) and one
                    // add, the same bits in both lanes since a + b == b + a
                    acc = acc + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0xb1, 0xf, 0xf, true));
                } else if constexpr (LPS > 1) {
                    // sub-block spans LPS lanes: fold their 16-term sums in lane order
                    const int first = lane - (li % LPS);
                    float tot = __shfl(acc, first, 64);
                    for (int k = 1; k < LPS; ++k) tot += __shfl(acc, first + k, 64);
                    acc = tot;
                }
                const float sse = T::round(acc);
                if (j == 0 || better(sse, best[sb])) {
                    best[sb] = sse;
                    jsel[s][sb] = j;
#pragma unroll
                    for (int i = 0; i < n; ++i) {
                        dsel[s][sb * n + i] = dj[sb * n + i];
                        sqsel[s][sb * n + i] = sqj[sb * n + i];
                        csel[s][sb * n + i] = cj[sb * n + i];
                    }
                }
            }
        }
    }

    sstar = 0;
    if constexpr (S == 2) {
        float e0 = T::round(block_row_sum(sqsel[0], li, lpb, lane_base));
        float e1 = T::round(block_row_sum(sqsel[S - 1], li, lpb, lane_base));
        sstar = better(e1, e0) ? 1 : 0;
    }
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        out[i] = (S == 2 && sstar) ? dsel[S - 1][i] : dsel[0][i];
        cout[i] = (S == 2 && sstar) ? csel[S - 1][i] : csel[0][i];
    }
    l1sel = (S == 2 && sstar) ? l1[S - 1] : l1[0];
#pragma unroll
    for (int sb = 0; sb < NSUBL; ++sb) jsel_out[sb] = (S == 2 && sstar) ? jsel[S - 1][sb] : jsel[0][sb];
}

}  // namespace hbq
