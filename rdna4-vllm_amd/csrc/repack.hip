// Load-time repack of int4 expert weights, with their scales and zero-points, into the
// fragment layout the gfx950 kernels stream. Op layout (moe_kernel.hip:7-17): w (E, N, K/8)
// int32, nibble j of word k/8 holds k = 8 * (k/8) + j; scales (E, N, G) fp16; zero-points
// (E, N/8, G) int32 (nibble n % 8 of word n / 8) or none (zero-point 8). G = K / 128.
//
// Fragment layout: per expert e and 16-row tile t (rows 16t .. 16t+15), G blocks of 1 KB and
// then the tile's metadata, G * 16 words (frag_tile_words(G) words a tile):
//   * block g's 16-byte lane l holds row 16t + (l % 16), words 16g + 4(l / 16) .. +3 (k in
//     [128g + 32 (l / 16), +32)): exactly the raw-nibble B operand of lane l for
//     v_mfma_*_16x16x128_f8f6f4, so a wave loads one fragment-group as one contiguous KB;
//   * metadata word r * G + g is row 16t + r, group g: the fp16 scale's bits in bits 0..15 and
//     the zero-point in bits 16..19. A row's groups are adjacent, so a decode lane reads the
//     scales and zero-points of its row's groups in one load, next to the tile's weights.
// The int4 words move as whole 16-byte words, so the repack is exact.
#include "grouped_params.h"

namespace w4a8 {
namespace {

// One thread per output 16-byte word: a fragment lane's 4 words, or 4 metadata words.
__global__ void __launch_bounds__(256) repack_fragments_kernel(const uint4* __restrict__ w,
                                                               const uint16_t* __restrict__ sc,
                                                               const uint32_t* __restrict__ zp,
                                                               int64_t total, int N, int G,
                                                               uint4* __restrict__ out) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= total) return;
    const int per_tile = 68 * G;                                  // 16-byte words a tile
    const int64_t et = o / per_tile;                              // e * (N / 16) + t
    const int in = (int)(o % per_tile);
    if (in < 64 * G) {
        const int g = in >> 6, l = in & 63;
        const int64_t row = et * 16 + (l & 15);                   // e * N + n
        // source: words 16g + 4q .. of the row, as 16-byte word index row * (4G) + 4g + q
        out[o] = w[row * (4 * (int64_t)G) + 4 * g + (l >> 4)];
        return;
    }
    const int nt = N / 16;
    const int64_t e = et / nt;
    uint32_t m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int f = 4 * (in - 64 * G) + i;                      // metadata word of the tile
        const int r = f / G, g = f % G;
        const int n = (int)(et % nt) * 16 + r;
        const uint32_t s = sc[(e * N + n) * G + g];
        const uint32_t z = zp ? (zp[(e * (N / 8) + n / 8) * G + g] >> (4 * (n % 8))) & 0xFu : 8u;
        m[i] = s | (z << 16);
    }
    out[o] = make_uint4(m[0], m[1], m[2], m[3]);
}

}  // namespace

int64_t fragments_words(int64_t E, int64_t N, int64_t K) {
    return E * (N / 16) * frag_tile_words((int)(K / kGroup));
}

int launch_repack_fragments(const int32_t* w, const void* scales, const int32_t* zeros,
                            int64_t E, int64_t N, int64_t K, int32_t* out, hipStream_t stream) {
    if (N % 16 != 0 || K % kGroup != 0) {
        set_error("repack: needs N % 16 == 0 and K % 128 == 0");
        return W4A8_ERR_INVALID;
    }
    const int64_t total = fragments_words(E, N, K) / 4;   // 16-byte words
    if (total == 0) return W4A8_OK;
    repack_fragments_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
        reinterpret_cast<const uint4*>(w), static_cast<const uint16_t*>(scales),
        reinterpret_cast<const uint32_t*>(zeros), total, (int)N, (int)(K / kGroup),
        reinterpret_cast<uint4*>(out));
    return check_launch("repack_fragments_kernel");
}

}  // namespace w4a8
