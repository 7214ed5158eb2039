// Instantiations of the vLLM-layout fused decode (packed_decode_impl.h) for K=16.
#include "packed_decode_impl.h"

namespace ck {
namespace pd {
CK_PD_DEFINE_LAUNCH_FOR_K(16)
}  // namespace pd
}  // namespace ck
