// zh_mv_other.hip -- Q3_K, IQ4_XS, F16 and F32 matvec kernel instantiations (zh_mv.h),
// and the mixed IQ4_XS / Q3_K launches of an MoE layer (routed and shared experts).
#include "zh_mv.h"

namespace zh {

MvKernel pick_mv_other(int fmt, int in, int out, int cols, int n) {
    switch (fmt) {
    case Q3_K: return pick<Q3_K, Q3_K, true>(in, out, cols, n);
    case IQ4_XS: return pick<IQ4_XS, IQ4_XS, true>(in, out, cols, n);
    case F16: return pick<F16, F16, false>(in, out, cols, n);
    case F32: return pick<F32, F32, false>(in, out, cols, n);
    default: return nullptr;
    }
}

// the fused gate/up + down launch: routed IQ4_XS experts (with a Q3_K or
// IQ4_XS shared expert); the polled down body is the generic one (rows of
// fewer than 1024 values), gate/up the fast path of one wavefront per row or
// the generic one
MoeFfnKernel pick_moe_ffn(int f1, int f2, int gate_cols, int down_cols) {
    if (f1 != IQ4_XS || team_width(down_cols) >= 64) return nullptr;
    const int tg = team_width(gate_cols);
    if (tg > 64) return nullptr;
    if (f2 == Q3_K) return tg == 64 ? moe_ffn_kernel<IQ4_XS, Q3_K, 64> : moe_ffn_kernel<IQ4_XS, Q3_K, 0>;
    if (f2 == IQ4_XS) return tg == 64 ? moe_ffn_kernel<IQ4_XS, IQ4_XS, 64> : moe_ffn_kernel<IQ4_XS, IQ4_XS, 0>;
    return nullptr;
}

MvKernel pick_mv_moe(int f1, int f2, int in, int out, int cols) {
    if (f1 == IQ4_XS && f2 == Q3_K) {
        if (in == IN_NORM && out == OUT_SWIGLU) return pick_two<IQ4_XS, Q3_K, IN_NORM, OUT_SWIGLU>(cols);
        if (in == IN_PLAIN && out == OUT_STORE) return pick_two<IQ4_XS, Q3_K, IN_PLAIN, OUT_STORE>(cols);
    }
    return nullptr;
}

}  // namespace zh
