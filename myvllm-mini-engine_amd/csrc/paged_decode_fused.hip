// Instantiations of the decode attention kernel with the fused prologue
// (the decode step's KV write, or q/k RMSNorm + RoPE + KV write, before
// attention), for every head dim with one 16-byte chunk per lane, tile,
// wave count and load kind.  Own translation unit: it compiles in parallel
// with paged_decode.hip.
#include "paged_decode_kernel.h"

namespace mvme {

template <typename T, int D, int G, int NW, bool STREAM>
void launch_decode_fused(const DecodeArgs& a, dim3 grid, bool page_uniform, hipStream_t s) {
    launch_decode_kernel<T, D, G, NW, STREAM, true>(a, grid, page_uniform, s);
}

#define MVME_FUSED_NW_S(T, D, G, NW, S) \
    template void launch_decode_fused<T, D, G, NW, S>(const DecodeArgs&, dim3, bool, hipStream_t);
#define MVME_FUSED_G(T, D, G)                         \
    MVME_FUSED_NW_S(T, D, G, kSplitWaves, false)      \
    MVME_FUSED_NW_S(T, D, G, kSplitWaves, true)       \
    MVME_FUSED_NW_S(T, D, G, kWholeWaves, false)      \
    MVME_FUSED_NW_S(T, D, G, kWholeWaves, true)
#define MVME_FUSED_D(T, D) MVME_FUSED_G(T, D, 1) MVME_FUSED_G(T, D, 2) MVME_FUSED_G(T, D, 4)
#define MVME_FUSED_T(T) MVME_FUSED_D(T, 16) MVME_FUSED_D(T, 32) MVME_FUSED_D(T, 64) MVME_FUSED_D(T, 128) \
    MVME_FUSED_D(T, 256)

MVME_FUSED_T(Half)
MVME_FUSED_T(BFloat16)

}  // namespace mvme
