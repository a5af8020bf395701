// Decode kernels for float K/V with head_dim 256.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<float, 256>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
