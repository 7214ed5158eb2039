// Instantiations of the any-K decode (packed_decode_masked.h) for rows padded to 512.
#include "packed_decode_masked.h"

namespace ck {
namespace pd {
CK_PD_DEFINE_MASKED_FOR_K(512)
}  // namespace pd
}  // namespace ck
