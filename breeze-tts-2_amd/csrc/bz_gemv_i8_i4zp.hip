// WF_I4ZP instances of the int8 matrix-core kernel (compiled on their own).
#include "bz_gemv_i8.h"

namespace bz {
int launch_i8_i4zp(const GemvParams& p, const Launch& l, hipStream_t st) { return launch_i8_m<WF_I4ZP>(p, l, st); }
}  // namespace bz
