// Kernel 3: pack V into per-block transposed, key-permuted MFMA tiles.
//
// The attention kernel computes O^T = Vt P^T on v_mfma_f32_32x32x16_bf16.
// Its A operand for k-step s (16 keys) and lane half h wants, for one head
// dimension row d, the 8 keys KEY(s,h,e) = 16s + 8(e/4) + 4h + e%4 (e=0..7)
// as one contiguous 16-byte chunk, because that is the order in which the
// S^T accumulators hold the probabilities. This kernel writes, per 64-key
// block, a [64 d][64 positions] tile with position 16s + 8h + e holding key
// KEY(s,h,e), zero padded past the sequence end. One 8 KB tile per block is
// read once and written once (HBM-bound, 16 KB of traffic per block).
// Precedent in the reference: TransposePadPermuteKernel
// (ZIP:csrc/fused/fused.cu:26-78), which permutes tokens for fp8 MMA.
#include "common.h"

namespace vasc {
namespace {

constexpr int kBlockK = 64;
constexpr int kHeadDim = 64;
constexpr int kPad = 8;  // LDS row padding (elements) against bank conflicts

__global__ __launch_bounds__(256) void pack_v_kernel(const uint16_t *__restrict__ v, int64_t sb, int64_t sh,
                                                     int64_t st, int64_t H, int64_t nk, int64_t nkb,
                                                     uint16_t *__restrict__ vt) {
  __shared__ uint16_t tile[kHeadDim][kBlockK + kPad];  // [d][key]
  const int64_t blk = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const uint16_t *src = v + b * sb + h * sh;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ci = tid + 256 * u;
    const int key = ci >> 3, dc = ci & 7;
    const int64_t tok = blk * kBlockK + key;
    u32x4 x = u32x4{0, 0, 0, 0};
    if (tok < nk) x = *reinterpret_cast<const u32x4 *>(src + tok * st + dc * 8);
    const uint16_t *e = reinterpret_cast<const uint16_t *>(&x);
#pragma unroll
    for (int i = 0; i < 8; ++i) tile[dc * 8 + i][key] = e[i];
  }
  __syncthreads();
  uint16_t *dst = vt + (bh * nkb + blk) * (kBlockK * kHeadDim);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int ci = tid + 256 * u;
    const int d = ci >> 3, chunk = ci & 7;
    const int s = chunk >> 1, hh = chunk & 1;
    uint16_t out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = tile[d][16 * s + 8 * (e >> 2) + 4 * hh + (e & 3)];
    *reinterpret_cast<u32x4 *>(dst + d * kBlockK + chunk * 8) = *reinterpret_cast<const u32x4 *>(out);
  }
}

}  // namespace
}  // namespace vasc

extern "C" int64_t vasc_packed_v_elems(int64_t B, int64_t H, int64_t nk, int64_t d) {
  if (B <= 0 || H <= 0 || nk <= 0 || d <= 0) return 0;
  return B * H * vasc::cdiv(nk, 64) * 64 * d;
}

extern "C" int vasc_pack_v(const uint16_t *v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t B, int64_t H,
                           int64_t nk, int64_t d, uint16_t *vt, void *stream) {
  VASC_SUPPORTED(d == 64, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(v != nullptr && vt != nullptr, "v and vt are required");
  VASC_REQUIRE(B > 0 && H > 0 && nk > 0, "sizes must be positive");
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15) == 0 && (reinterpret_cast<uintptr_t>(vt) & 15) == 0,
               "v and vt must be 16-byte aligned");
  VASC_REQUIRE(v_sb % 8 == 0 && v_sh % 8 == 0 && v_st % 8 == 0 && v_sb >= 0 && v_sh >= 0 && v_st > 0,
               "v strides must be non-negative multiples of 8 elements");
  const int64_t nkb = vasc::cdiv(nk, 64);
  VASC_REQUIRE(nkb < (int64_t(1) << 31) && B * H < 65536, "grid too large");
  hipLaunchKernelGGL(vasc::pack_v_kernel, dim3(nkb, B * H), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), v,
                     v_sb, v_sh, v_st, H, nk, nkb, vt);
  return vasc::check_launch("vasc_pack_v");
}
