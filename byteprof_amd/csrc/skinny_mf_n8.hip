// The matrix-core skinny kernel for launches whose waves have exactly 8 K segments each (skinny_mf_kernel.h).
#define BP_MF_INSTANTIATE
#include "skinny_mf_kernel.h"

namespace bp {
template MfFn mf_pick_n<8>(int, int, int, int, bool, int, bool, bool, int);
}  // namespace bp
