// gemv_f4.hip -- decode kernel instantiations for weight format 4.
#include "gemv_impl.hpp"

namespace grim {
GRIM_DECODE_INSTANTIATE(4)
}  // namespace grim
