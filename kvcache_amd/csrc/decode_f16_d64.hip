// Decode kernels for _Float16 K/V with head_dim 64.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<_Float16, 64>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
