// gemv_f0.hip -- decode kernel instantiations for weight format 0.
#include "gemv_impl.hpp"

namespace grim {
GRIM_DECODE_INSTANTIATE(0)
}  // namespace grim
