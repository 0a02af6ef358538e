// Load-time repack of int4 expert weights into the fragment layout the gfx950 kernels
// stream. Op layout (moe_kernel.hip:7-17): w (E, N, K/8) int32, nibble j of word k/8 holds
// k = 8 * (k/8) + j. Fragment layout: for expert e, 16-row tile t (rows 16t .. 16t+15) and
// 128-wide K group g, one 1 KB block; its 16-byte lane l holds row 16t + (l % 16), words
// 16g + 4(l / 16) .. +3 (k in [128g + 32 (l / 16), +32)): exactly the raw-nibble B operand
// of lane l for v_mfma_*_16x16x128_f8f6f4. A wave therefore loads one fragment-group as one
// contiguous kilobyte. Blocks are ordered (e, t, g). The permutation moves whole 16-byte
// words, so it is exact; scales and zero-points keep the op layout.
#include "grouped_params.h"

namespace w4a8 {
namespace {

__global__ void __launch_bounds__(256) repack_fragments_kernel(const uint4* __restrict__ w,
                                                               int64_t total, int nt, int G,
                                                               uint4* __restrict__ out) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;   // output 16-byte word
    if (o >= total) return;
    const int l = (int)(o & 63);
    const int64_t blk = o >> 6;                                   // (e * nt + t) * G + g
    const int g = (int)(blk % G);
    const int64_t et = blk / G;                                   // e * nt + t
    const int64_t row = et * 16 + (l & 15);                       // e * N + n
    // source: words 16g + 4q .. of the row, as 16-byte word index row * (4G) + 4g + q
    out[o] = w[row * (4 * (int64_t)G) + 4 * g + (l >> 4)];
}

}  // namespace

int launch_repack_fragments(const int32_t* w, int64_t E, int64_t N, int64_t K, int32_t* out,
                            hipStream_t stream) {
    if (N % 16 != 0 || K % kGroup != 0) {
        set_error("repack: needs N % 16 == 0 and K % 128 == 0");
        return W4A8_ERR_INVALID;
    }
    const int64_t total = E * N * K / 32;   // 16-byte words (32 nibbles each)
    if (total == 0) return W4A8_OK;
    const int G = (int)(K / kGroup);
    repack_fragments_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(w), total, (int)(N / 16), G, reinterpret_cast<uint4*>(out));
    return check_launch("repack_fragments_kernel");
}

}  // namespace w4a8
