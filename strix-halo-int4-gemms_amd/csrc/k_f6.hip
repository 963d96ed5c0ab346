// GEMM kernels of the fp6 path (shk_f6.h): the 256x256 per-channel tile and
// the 256x128 SwiGLU tile.  They read operands already converted to the
// block format, so one instantiation serves every layout; the table holds
// one entry per layout (NN, NT, TN), which differ in how the operands are
// converted.  Compiled with the iterative ILP scheduler, which keeps the 256
// accumulators in place (k_dense.hip).
#include "shk_table.h"

namespace shk {
namespace {

template <int BN, bool SWIGLU>
using C = Cfg<4, true, true, 256, BN, 128, 2, 2, SWIGLU, false, 64, false, 0>;

}  // namespace

void append_dense_f6(std::vector<Entry>& t, int layout) {
  t.push_back(f6_entry<C<256, false>>(layout));
  t.push_back(f6_entry<C<128, true>>(layout));
}

}  // namespace shk
