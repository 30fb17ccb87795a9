// gemv_f64.hip -- decode kernel instantiations for weight format 64.
#include "gemv_impl.hpp"

namespace grim {
GRIM_DECODE_INSTANTIATE(64)
}  // namespace grim
