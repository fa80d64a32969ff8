// zh_mv_q8.hip -- Q8_0 matvec kernel instantiations (zh_mv.h).
#include "zh_mv.h"

namespace zh {

MvKernel pick_mv_q8_0(int in, int out, int cols, int n) { return pick<Q8_0, Q8_0, true>(in, out, cols, n); }

}  // namespace zh
