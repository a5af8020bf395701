// Decode kernels for _Float16 K/V with head_dim 256.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<_Float16, 256>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
