// Decode kernels for float K/V with head_dim 64.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<float, 64>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
