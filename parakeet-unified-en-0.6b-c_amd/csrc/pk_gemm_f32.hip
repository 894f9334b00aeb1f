// pk_gemm_f32.hip - instantiates the tile kernels for W_F32 weights.
#include "pk_gemm_tiles.h"

namespace pkgpu {
namespace tiles {

hipError_t launch_chain_f32(int cfg, const KArgs& a, hipStream_t s)
{
    return launch_chain<W_F32>(cfg, a, s);
}

}  // namespace tiles
}  // namespace pkgpu
