// float16/bfloat16 GEMM with operands fetched straight into LDS (the kernel
// is in gemm_dma.h): eligibility, and the 256x256 instantiations.
#include "gemm_dma.h"

namespace tvk {

bool dma_applies(const GemmArgs& p, bool a_kmajor, bool b_kmajor) {
    // K off the 32 grid: the last k step runs whole, so its loads past K must read zeros
    if (p.K < D_BK || (p.K % D_BK != 0 && !p.kzero)) return false;
    auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
    if (!al16(p.a) || !al16(p.b)) return false;
    if (p.batch > 1 && (p.sa[0] % 8 != 0 || p.sb[0] % 8 != 0)) return false;
    if (p.bh > 1 && (p.sa_h % 8 != 0 || p.sb_h % 8 != 0)) return false;
    // every 16-byte chunk starts 16-byte aligned: the stride between the rows
    // of the contiguous dimension is a multiple of 8 elements
    const int64_t a_rows = a_kmajor ? p.sa[1] : p.sa[2];
    const int64_t b_rows = b_kmajor ? p.sb[2] : p.sb[1];
    if ((a_kmajor ? p.M : p.K) > 1 && a_rows % 8 != 0) return false;
    if ((b_kmajor ? p.N : p.K) > 1 && b_rows % 8 != 0) return false;
    // an m/n-contiguous operand whose last chunk straddled M or N would lose
    // the valid part of that chunk on the last k-row: the range check ends
    // the buffer at the last element, and extending it would read memory the
    // tensor may not own
    if (!a_kmajor && p.M % 8 != 0) return false;
    if (!b_kmajor && p.N % 8 != 0) return false;
    return true;
}

hipError_t launch_dma(int dtype, GemmArgs& p, bool a_kmajor, bool b_kmajor, int tile, hipStream_t s, int stages) {
    if (tile == DMA_TILE_128X256 || tile == DMA_TILE_256X128) {
        launch_dma_rect(dtype, p, a_kmajor, b_kmajor, s, tile == DMA_TILE_128X256);
        return hipGetLastError();
    }
    if (dtype == TVK_F16) {
        if (tile == 256) launch_dma_tile<TVK_F16, 256, 256, 4>(p, a_kmajor, b_kmajor, s);
        else launch_dma128(dtype, p, a_kmajor, b_kmajor, s, stages);
    } else {
        if (tile == 256) launch_dma_tile<TVK_BF16, 256, 256, 4>(p, a_kmajor, b_kmajor, s);
        else launch_dma128(dtype, p, a_kmajor, b_kmajor, s, stages);
    }
    return hipGetLastError();
}

}  // namespace tvk
