// gemv_f3.hip -- decode kernel instantiations for weight format 3.
#include "gemv_impl.hpp"

namespace grim {
GRIM_DECODE_INSTANTIATE(3)
}  // namespace grim
