// pk_gemm_i4.hip - instantiates the tile kernels for W_I4 weights.
#include "pk_gemm_tiles.h"

namespace pkgpu {
namespace tiles {

hipError_t launch_chain_i4(int cfg, const KArgs& a, hipStream_t s)
{
    return launch_chain<W_I4>(cfg, a, s);
}

}  // namespace tiles
}  // namespace pkgpu
