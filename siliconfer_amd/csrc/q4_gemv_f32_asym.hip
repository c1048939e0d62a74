// Block-layout GEMV launches for f32 activations, asymmetric codes (one file per pair: compile time).
#include "q4_gemv_blk.h"

namespace sf_gemv {
template void launch_blk<SF_F32, true>(const BlkPlan &, const GemvArgs &, int, const float *, float,
                                      const SfRopeAppend *, const int *);
}  // namespace sf_gemv
