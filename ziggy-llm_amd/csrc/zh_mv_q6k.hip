// zh_mv_q6k.hip -- Q6_K matvec kernel instantiations (zh_mv.h).
#include "zh_mv.h"

namespace zh {

MvKernel pick_mv_q6k(int in, int out, int cols, int n) { return pick<Q6_K, Q6_K, true>(in, out, cols, n); }

}  // namespace zh
