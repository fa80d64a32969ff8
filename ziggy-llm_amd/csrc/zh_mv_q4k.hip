// zh_mv_q4k.hip -- Q4_K matvec kernel instantiations (zh_mv.h), and the mixed
// Q4_K / Q6_K q/k/v launch of a Q4_K_M layer.
#include "zh_mv.h"

namespace zh {

MvKernel pick_mv_q4k(int in, int out, int cols, int n) { return pick<Q4_K, Q4_K, true>(in, out, cols, n); }

MvKernel pick_mv_mixed(int f1, int f2, int cols, int n) {
    if (f1 == Q4_K && f2 == Q6_K) return pick_mixed<Q4_K, Q6_K>(cols, n);
    if (f1 == Q6_K && f2 == Q4_K) return pick_mixed<Q6_K, Q4_K>(cols, n);
    return nullptr;
}

}  // namespace zh
