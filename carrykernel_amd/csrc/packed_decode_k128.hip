// Instantiations of the vLLM-layout fused decode (packed_decode_impl.h) for K=128.
#include "packed_decode_impl.h"

namespace ck {
namespace pd {
CK_PD_DEFINE_LAUNCH_FOR_K(128)
}  // namespace pd
}  // namespace ck
