// zh_mv_other.hip -- Q3_K, IQ4_XS, F16 and F32 matvec kernel instantiations (zh_mv.h).
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

}  // namespace zh
