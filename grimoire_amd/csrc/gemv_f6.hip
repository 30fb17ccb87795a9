// gemv_f6.hip -- decode kernel instantiations for weight format 6.
#include "gemv_impl.hpp"

namespace grim {
GRIM_DECODE_INSTANTIATE(6)
}  // namespace grim
