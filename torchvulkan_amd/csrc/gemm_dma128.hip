// The 128x128-tile (and 128x256 / 256x128) instantiations of the LDS-ring
// GEMM kernel (gemm_dma.h), built with the MFMA results in VGPRs.
#include "gemm_dma.h"

namespace tvk {

void launch_dma128(int dtype, GemmArgs& p, bool a_kmajor, bool b_kmajor, hipStream_t s, int stages) {
    if (dtype == TVK_F16) {
        if (stages == 8) launch_dma_tile<TVK_F16, 128, 128, 8>(p, a_kmajor, b_kmajor, s);
        else launch_dma_tile<TVK_F16, 128, 128, 4>(p, a_kmajor, b_kmajor, s);
    } else {
        if (stages == 8) launch_dma_tile<TVK_BF16, 128, 128, 8>(p, a_kmajor, b_kmajor, s);
        else launch_dma_tile<TVK_BF16, 128, 128, 4>(p, a_kmajor, b_kmajor, s);
    }
}

void launch_dma_rect(int dtype, GemmArgs& p, bool a_kmajor, bool b_kmajor, hipStream_t s, bool wide) {
    if (dtype == TVK_F16) {
        if (wide) launch_dma_tile<TVK_F16, 128, 256, 4>(p, a_kmajor, b_kmajor, s);
        else launch_dma_tile<TVK_F16, 256, 128, 4>(p, a_kmajor, b_kmajor, s);
    } else {
        if (wide) launch_dma_tile<TVK_BF16, 128, 256, 4>(p, a_kmajor, b_kmajor, s);
        else launch_dma_tile<TVK_BF16, 256, 128, 4>(p, a_kmajor, b_kmajor, s);
    }
}

}  // namespace tvk
