// Decode kernels for float K/V with head_dim 128.
#include "decode_kernels.hpp"

namespace kvc {
template int launch_decode_d<float, 128>(const DecodeLaunch&, hipStream_t);
}  // namespace kvc
