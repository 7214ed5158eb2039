// Instantiations of the any-K decode (packed_decode_masked.h) for rows padded to 1024.
#include "packed_decode_masked.h"

namespace ck {
namespace pd {
CK_PD_DEFINE_MASKED_FOR_K(1024)
}  // namespace pd
}  // namespace ck
