// Decode kernels for float K/V with head_dim 32.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<float, 32>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
