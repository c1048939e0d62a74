// q4_gemv_bf16.hip — GEMV instantiations for bf16 activations (kernel in q4_gemv_kernel.h;
// one translation unit per activation type keeps the build parallel).
#include "q4_gemv_kernel.h"

namespace sf_gemv {
template void launch_x<SF_BF16>(const GemvPlan &, const GemvArgs &);
template void launch_pre<SF_BF16>(const GemvPlan &, const GemvArgs &, int, const float *, float);
template void launch_pre_rope<SF_BF16>(const GemvPlan &, const GemvArgs &, const float *, float,
                                      const SfRopeAppend &, const int *);
}  // namespace sf_gemv
