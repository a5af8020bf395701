// decode.hip -- decode launch dispatch over element type and head_dim.  The
// kernels live in decode_kernels.hpp; each (type, head_dim) pair is compiled in
// its own translation unit (decode_<type>_d<D>.hip) so the instantiations build
// in parallel.
#include "internal.hpp"
#include "kvc_abi.h"

namespace kvc {

namespace {
template <typename T>
int launch_typed(const DecodeLaunch& L, hipStream_t st) {
    switch (L.D) {
        case 32:  return launch_decode_d<T, 32>(L, st);
        case 64:  return launch_decode_d<T, 64>(L, st);
        case 128: return launch_decode_d<T, 128>(L, st);
        case 256: return launch_decode_d<T, 256>(L, st);
        default: return set_error(KVC_ERR_UNSUPPORTED, "head_dim must be 32, 64, 128 or 256");
    }
}
}  // namespace

int launch_decode(const DecodeLaunch& L, hipStream_t stream) {
    if (L.dtype == KVC_F16) return launch_typed<_Float16>(L, stream);
    if (L.dtype == KVC_F32) return launch_typed<float>(L, stream);
    return set_error(KVC_ERR_ARG, "dtype must be KVC_F32 or KVC_F16");
}

}  // namespace kvc
