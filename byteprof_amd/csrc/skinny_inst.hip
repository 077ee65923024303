// One (weight kind, activation-row bucket) slice of the skinny kernel menu. The build compiles this file once per
// slice with -DBP_KIND=<0 bf16 | 1 int8> -DBP_MT=<1|2|4|8|16>, so the slices compile in parallel.
#include "skinny_kernel.h"

#if !defined(BP_KIND) || !defined(BP_MT)
#error "compile with -DBP_KIND=<kind> -DBP_MT=<rows>"
#endif

namespace bp {
template SkinnyFn skinny_pick<BP_KIND, BP_MT>(int rows, int waves, bool vec);
}  // namespace bp
