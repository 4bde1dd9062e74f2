// Runner op: the residual update and LayerNorm between the sub-layers of the
// VGGT/Pi3-shaped blocks (no counterpart in the sparse-attention path; the
// benchmark's aggregator forward uses it).
//
// One wave per token row of `dim` bf16 features (dim = 512 V, 8 features per
// lane per 16-byte chunk). s = bf16(x + bf16(y * gamma)) is what torch's bf16
// LayerScale multiply and residual add produce (each product and sum in
// fp32, rounded to bf16); the LayerNorm of s is computed in fp32 with the
// mean and variance as wave sums and written as bf16((s - mean) * rstd * w +
// b). The row is read once and its two results written once: 4 row-sized
// transfers instead of the 8 of the separate multiply, add and norm kernels.
#include "common.h"
#include "../../include/vasc_runner.h"

namespace vasc {
namespace {

struct ResNormParams {
  const uint16_t *x, *y;
  int64_t ldx, ldy;
  const uint16_t *gamma;  // [dim] LayerScale, or NULL
  const uint16_t *w, *b;  // [dim] LayerNorm affine (each may be NULL)
  float eps;
  uint16_t *x_out;
  int64_t ldo;
  uint16_t *n_out;  // LayerNorm of the updated row, or NULL
  int64_t ldn;
  int64_t rows;
};

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int V>
__global__ __launch_bounds__(256) void residual_norm_kernel(const ResNormParams p) {
  constexpr int kDim = 512 * V;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  u32x4 xr[V], yr[V], gr[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = (v * 64 + lane) * 8;
    xr[v] = *reinterpret_cast<const u32x4 *>(p.x + row * p.ldx + c);
    yr[v] = *reinterpret_cast<const u32x4 *>(p.y + row * p.ldy + c);
    gr[v] = p.gamma ? *reinterpret_cast<const u32x4 *>(p.gamma + c) : u32x4{0, 0, 0, 0};
  }
  float s[V][8];
#pragma unroll
  for (int v = 0; v < V; ++v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sh = (e & 1) ? 16u : 0u;
      const float xv = bf16_to_f32(static_cast<uint16_t>(xr[v][e >> 1] >> sh));
      float yv = bf16_to_f32(static_cast<uint16_t>(yr[v][e >> 1] >> sh));
      if (p.gamma) yv = round_bf16(yv * bf16_to_f32(static_cast<uint16_t>(gr[v][e >> 1] >> sh)));
      s[v][e] = round_bf16(xv + yv);
    }
  }
  if (p.x_out) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(s[v][2 * e], s[v][2 * e + 1]);
      *reinterpret_cast<u32x4 *>(p.x_out + row * p.ldo + (v * 64 + lane) * 8) = o;
    }
  }
  if (!p.n_out) return;
  float sum = 0.f;
#pragma unroll
  for (int v = 0; v < V; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += s[v][e];
  const float mean = wave_sum_f32(sum) / static_cast<float>(kDim);
  float sq = 0.f;
#pragma unroll
  for (int v = 0; v < V; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) sq += (s[v][e] - mean) * (s[v][e] - mean);
  const float rstd = 1.0f / sqrtf(wave_sum_f32(sq) / static_cast<float>(kDim) + p.eps);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = (v * 64 + lane) * 8;
    const u32x4 wr = p.w ? *reinterpret_cast<const u32x4 *>(p.w + c) : u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    const u32x4 br = p.b ? *reinterpret_cast<const u32x4 *>(p.b + c) : u32x4{0, 0, 0, 0};
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t sh = k ? 16u : 0u;
        const float wv = bf16_to_f32(static_cast<uint16_t>(wr[e] >> sh));
        const float bv = bf16_to_f32(static_cast<uint16_t>(br[e] >> sh));
        r[k] = ((s[v][2 * e + k] - mean) * rstd) * wv + bv;
      }
      o[e] = pack_bf16x2(r[0], r[1]);
    }
    *reinterpret_cast<u32x4 *>(p.n_out + row * p.ldn + c) = o;
  }
}

int check_rows(const char *name, const void *ptr, int64_t ld, int64_t dim, bool required) {
  if (!ptr) {
    VASC_REQUIRE(!required, "%s is NULL", name);
    return VASC_OK;
  }
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(ptr) & 15) == 0, "%s must be 16-byte aligned", name);
  VASC_REQUIRE(ld >= dim && ld % 8 == 0, "%s row stride %lld must be a multiple of 8 and at least dim %lld", name,
               (long long)ld, (long long)dim);
  return VASC_OK;
}

}  // namespace
}  // namespace vasc

extern "C" int vasc_residual_norm(const uint16_t *x, int64_t ldx, const uint16_t *y, int64_t ldy,
                                  const uint16_t *gamma, const uint16_t *norm_w, const uint16_t *norm_b,
                                  float eps, uint16_t *x_out, int64_t ldo, uint16_t *norm_out, int64_t ldn,
                                  int64_t rows, int64_t dim, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(dim == 512 || dim == 1024 || dim == 1536 || dim == 2048, "dim %lld not built (512, 1024, 1536, 2048)",
                 (long long)dim);
  VASC_REQUIRE(rows > 0, "rows must be positive");
  VASC_REQUIRE(x_out || norm_out, "x_out and norm_out are both NULL");
  int rc;
  if ((rc = check_rows("x", x, ldx, dim, true))) return rc;
  if ((rc = check_rows("y", y, ldy, dim, true))) return rc;
  if ((rc = check_rows("x_out", x_out, ldo, dim, false))) return rc;
  if ((rc = check_rows("norm_out", norm_out, ldn, dim, false))) return rc;
  for (const uint16_t *v : {gamma, norm_w, norm_b})
    VASC_REQUIRE((reinterpret_cast<uintptr_t>(v) & 15) == 0, "gamma and the norm parameters must be 16-byte aligned");
  VASC_REQUIRE(eps >= 0.f, "eps must be non-negative");
  VASC_REQUIRE(rows < (int64_t(1) << 32), "too many rows");
  ResNormParams p;
  p.x = x; p.ldx = ldx; p.y = y; p.ldy = ldy;
  p.gamma = gamma; p.w = norm_w; p.b = norm_b; p.eps = eps;
  p.x_out = x_out; p.ldo = ldo; p.n_out = norm_out; p.ldn = ldn;
  p.rows = rows;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(cdiv(rows, 4)));
  switch (dim) {
    case 512: hipLaunchKernelGGL(residual_norm_kernel<1>, grid, dim3(256), 0, s, p); break;
    case 1024: hipLaunchKernelGGL(residual_norm_kernel<2>, grid, dim3(256), 0, s, p); break;
    case 1536: hipLaunchKernelGGL(residual_norm_kernel<3>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(residual_norm_kernel<4>, grid, dim3(256), 0, s, p); break;
  }
  return check_launch("vasc_residual_norm");
}
