// Kernel 1: block mean pooling of Q/K/V, pair innovation, pooled softmax.
//
// 1a (pool_qkv_kernel) is HBM-bound: each workgroup streams one 128-token
// span of Q, K and V (3 x 16 KB) with 16-byte coalesced loads, reduces the
// 8-lane groups that share a 16-byte column with xor shuffles and the four
// waves through LDS, and writes one pooled Q row, two pooled K rows and two
// pooled V rows (bf16, as avg_pool1d on bf16 input produces), plus the
// innovation of the V pair it just pooled, so the value-contrast score needs
// no second pass over V. Algorithmic traffic: 3*2*d bytes per token read,
// (2*d*(1/128 + 2/64)) + 4/128 bytes per token written.
//
// 1b (pooled_softmax_kernel) computes the pooled logits on MFMA with the
// transposed-output trick (one lane = one query row) in two passes (online
// max/sum, then normalised write). Its cost is the fp32 write of the
// [Qb, Kb] probability matrix.
//
// Reference: predict_attention (attention.py:31-104),
// _mean_pool_contiguous_value_blocks (sparse_wrapper.py:2839-2861),
// pair innovation (sparse_wrapper.py:3733-3740).
#include "innovation.h"

namespace vasc {
namespace {

constexpr int kHeadDim = 64;

struct PoolParams {
  const uint16_t *x[3];
  int64_t sb[3], sh[3], st[3];
  int64_t ntok[3];   // tokens of q, k, v
  int64_t nblk[3];   // pooled blocks of q, k, v
  uint16_t *out[3];  // pooled q, k, v
  float *innovation;
  int64_t H, npairs;
};

__global__ __launch_bounds__(256) void pool_qkv_kernel(const PoolParams p) {
  __shared__ float red[3][2][4][kHeadDim];
  __shared__ float pv[2][kHeadDim];
  const int64_t chunk = blockIdx.x;  // 128-token span
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int dc = tid & 7, r = tid >> 3;

  // Issue all 12 row loads (3 tensors x 4 rows) before any reduction so each
  // thread keeps 192 bytes in flight.
  u32x4 raw[3][4];
#pragma unroll
  for (int X = 0; X < 3; ++X) {
    const uint16_t *src = p.x[X] ? p.x[X] + b * p.sb[X] + h * p.sh[X] + dc * 8 : nullptr;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t tok = chunk * 128 + r + 32 * u;
      raw[X][u] = (src && tok < p.ntok[X]) ? *reinterpret_cast<const u32x4 *>(src + tok * p.st[X])
                                           : u32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int X = 0; X < 3; ++X) {
    if (p.x[X] == nullptr) continue;
    float acc[2][8];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[half][i] = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[u >> 1][2 * i] += __uint_as_float(raw[X][u][i] << 16);
        acc[u >> 1][2 * i + 1] += __uint_as_float(raw[X][u][i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float s = acc[half][i];
        s += __shfl_xor(s, 8);
        s += __shfl_xor(s, 16);
        s += __shfl_xor(s, 32);
        acc[half][i] = s;
      }
    if (lane < 8) {
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int i = 0; i < 8; ++i) red[X][half][w][dc * 8 + i] = acc[half][i];
    }
  }
  __syncthreads();

  // Finalise: q -> one 128-token block; k, v -> two 64-token blocks.
  for (int item = tid; item < 5 * kHeadDim; item += 256) {
    const int d = item & 63;
    const int slot = item >> 6;  // 0: q, 1-2: k blocks, 3-4: v blocks
    const int X = slot == 0 ? 0 : (slot <= 2 ? 1 : 2);
    if (p.x[X] == nullptr) continue;
    float sum;
    int64_t blk, count;
    if (X == 0) {
      sum = ((red[0][0][0][d] + red[0][0][1][d]) + (red[0][0][2][d] + red[0][0][3][d])) +
            ((red[0][1][0][d] + red[0][1][1][d]) + (red[0][1][2][d] + red[0][1][3][d]));
      blk = chunk;
      count = p.ntok[0] - chunk * 128;
      count = count > 128 ? 128 : count;
    } else {
      const int half = (slot - 1) & 1;
      sum = (red[X][half][0][d] + red[X][half][1][d]) + (red[X][half][2][d] + red[X][half][3][d]);
      blk = 2 * chunk + half;
      count = p.ntok[X] - blk * 64;
      count = count > 64 ? 64 : count;
    }
    if (count <= 0) continue;
    const uint16_t mean = f32_to_bf16(sum / static_cast<float>(count));
    p.out[X][(bh * p.nblk[X] + blk) * kHeadDim + d] = mean;
    if (X == 2) pv[slot - 3][d] = bf16_to_f32(mean);
  }
  if (p.innovation == nullptr) return;
  __syncthreads();
  if (w == 0 && chunk < p.npairs) {
    const float lv = pv[0][lane];
    const float rv = (2 * chunk + 1 < p.nblk[2]) ? pv[1][lane] : lv;
    const float iota = pair_innovation_wave(lv, rv);
    if (lane == 0) p.innovation[bh * p.npairs + chunk] = iota;
  }
}

__global__ __launch_bounds__(256) void pair_innovation_kernel(const float *__restrict__ v, int64_t kb,
                                                              int64_t npairs, int64_t total,
                                                              float *__restrict__ out) {
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (pair >= total) return;
  const int lane = threadIdx.x & 63;
  const int64_t bh = pair / npairs, pp = pair % npairs;
  const float *base = v + bh * kb * kHeadDim;
  const float lv = base[(2 * pp) * kHeadDim + lane];
  const float rv = (2 * pp + 1 < kb) ? base[(2 * pp + 1) * kHeadDim + lane] : lv;
  const float iota = pair_innovation_wave(lv, rv);
  if (lane == 0) out[pair] = iota;
}

__device__ __forceinline__ floatx16 mfma32(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Logits of one 32-key tile against the wave's 32 pooled query rows.
// Returns acc[r] for key 32t + 8(r/4) + 4hf + r%4 and query row lane%32.
__device__ __forceinline__ floatx16 pooled_tile(const uint16_t *pk, int64_t kb, int64_t t, const u32x4 *qf,
                                                int lr, int hf, float scale, bool round) {
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  const int64_t key = 32 * t + lr;
  const bool ok = key < kb;
  const uint16_t *row = pk + (ok ? key : 0) * kHeadDim;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const u32x4 a = ok ? *reinterpret_cast<const u32x4 *>(row + 16 * s + 8 * hf) : u32x4{0, 0, 0, 0};
    acc = mfma32(a, qf[s], acc);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t kk = 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
    float x = acc[r];
    x = round ? round_bf16(round_bf16(x) * scale) : x * scale;
    acc[r] = kk < kb ? x : -INFINITY;
  }
  return acc;
}

constexpr int kSoftmaxWaves = 16;  // key tiles of one 32-row strip spread over 16 waves

__global__ __launch_bounds__(kSoftmaxWaves * 64) void pooled_softmax_kernel(const uint16_t *__restrict__ pq,
                                                                           const uint16_t *__restrict__ pk,
                                                                           int64_t qb, int64_t kb, float scale,
                                                                           int round, float *__restrict__ prob) {
  __shared__ float sm_m[kSoftmaxWaves][32];
  __shared__ float sm_s[kSoftmaxWaves][32];
  const int64_t bh = blockIdx.y;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lr = l & 31, hf = l >> 5;
  const int64_t qrow = row0 + lr;
  const bool qok = qrow < qb;
  const uint16_t *qbase = pq + (bh * qb + (qok ? qrow : 0)) * kHeadDim;
  const uint16_t *kbase = pk + bh * kb * kHeadDim;
  u32x4 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = qok ? *reinterpret_cast<const u32x4 *>(qbase + 16 * s + 8 * hf) : u32x4{0, 0, 0, 0};
  const int64_t ntiles = cdiv(kb, 32);

  float m = -INFINITY, sum = 0.f;
  for (int64_t t = w; t < ntiles; t += kSoftmaxWaves) {
    const floatx16 x = pooled_tile(kbase, kb, t, qf, lr, hf, scale, round != 0);
    float mx = x[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, x[r]);
    const float mn = fmaxf(m, mx);
    if (mn == -INFINITY) continue;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += expf(x[r] - mn);
    sum = sum * expf(m - mn) + s;
    m = mn;
  }
  {  // merge the two lanes of each row
    const float mo = __shfl_xor(m, 32), so = __shfl_xor(sum, 32);
    const float mn = fmaxf(m, mo);
    sum = (m == -INFINITY ? 0.f : sum * expf(m - mn)) + (mo == -INFINITY ? 0.f : so * expf(mo - mn));
    m = mn;
  }
  if (hf == 0) {
    sm_m[w][lr] = m;
    sm_s[w][lr] = sum;
  }
  __syncthreads();
  float gm = -INFINITY;
#pragma unroll
  for (int i = 0; i < kSoftmaxWaves; ++i) gm = fmaxf(gm, sm_m[i][lr]);
  float gs = 0.f;
#pragma unroll
  for (int i = 0; i < kSoftmaxWaves; ++i) {
    const float mi = sm_m[i][lr];
    if (mi != -INFINITY) gs += sm_s[i][lr] * expf(mi - gm);
  }
  const float inv = 1.f / gs;
  // Lanes of padding rows stay: they feed key rows to the MFMA A operand.
  float *out = prob + (bh * qb + (qok ? qrow : 0)) * kb;
  for (int64_t t = w; t < ntiles; t += kSoftmaxWaves) {
    const floatx16 x = pooled_tile(kbase, kb, t, qf, lr, hf, scale, round != 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t kk = 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (qok && kk < kb) out[kk] = expf(x[r] - gm) * inv;
    }
  }
}

}  // namespace
}  // namespace vasc

extern "C" int vasc_pool_qkv(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const uint16_t *k,
                             int64_t k_sb, int64_t k_sh, int64_t k_st, const uint16_t *v, int64_t v_sb,
                             int64_t v_sh, int64_t v_st, int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d,
                             int64_t block_q, int64_t block_k, uint16_t *pooled_q, uint16_t *pooled_k,
                             uint16_t *pooled_v, float *innovation, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == 64 && block_q == 128 && block_k == 64,
                 "pooling variant d=%lld block_q=%lld block_k=%lld not built (built: 64/128/64)", (long long)d,
                 (long long)block_q, (long long)block_k);
  VASC_REQUIRE(B > 0 && H > 0, "B and H must be positive");
  VASC_REQUIRE(q || k || v, "nothing to pool");
  VASC_REQUIRE(!q || (pooled_q && nq > 0), "q needs pooled_q and nq > 0");
  VASC_REQUIRE(!k || (pooled_k && nk > 0), "k needs pooled_k and nk > 0");
  VASC_REQUIRE(!v || (pooled_v && nk > 0), "v needs pooled_v and nk > 0");
  VASC_REQUIRE(!innovation || v, "innovation needs v");
  const uint16_t *xs[3] = {q, k, v};
  const int64_t strides[3][3] = {{q_sb, q_sh, q_st}, {k_sb, k_sh, k_st}, {v_sb, v_sh, v_st}};
  PoolParams p;
  for (int X = 0; X < 3; ++X) {
    p.x[X] = xs[X];
    p.sb[X] = strides[X][0];
    p.sh[X] = strides[X][1];
    p.st[X] = strides[X][2];
    if (xs[X]) {
      VASC_REQUIRE((reinterpret_cast<uintptr_t>(xs[X]) & 15) == 0, "input %d must be 16-byte aligned", X);
      VASC_REQUIRE(p.sb[X] % 8 == 0 && p.sh[X] % 8 == 0 && p.st[X] % 8 == 0 && p.sb[X] >= 0 && p.sh[X] >= 0 &&
                       p.st[X] > 0,
                   "input %d strides must be non-negative multiples of 8 elements", X);
    }
  }
  p.ntok[0] = nq;
  p.ntok[1] = nk;
  p.ntok[2] = nk;
  p.nblk[0] = cdiv(nq, 128);
  p.nblk[1] = cdiv(nk, 64);
  p.nblk[2] = cdiv(nk, 64);
  p.out[0] = pooled_q;
  p.out[1] = pooled_k;
  p.out[2] = pooled_v;
  p.innovation = innovation;
  p.H = H;
  p.npairs = cdiv(p.nblk[2], 2);
  const int64_t chunks = cdiv(q ? nq : 0, 128) > cdiv(nk, 128) ? cdiv(nq, 128) : cdiv(nk, 128);
  VASC_REQUIRE(chunks < (int64_t(1) << 31) && B * H < 65536, "grid too large");
  hipLaunchKernelGGL(pool_qkv_kernel, dim3(chunks, B * H), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
  return check_launch("vasc_pool_qkv");
}

extern "C" int vasc_pair_innovation(const float *pooled_v, int64_t B, int64_t H, int64_t kb, int64_t d,
                                    float *innovation, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == 64, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(pooled_v && innovation && B > 0 && H > 0 && kb > 0, "invalid arguments");
  const int64_t npairs = cdiv(kb, 2);
  const int64_t total = B * H * npairs;
  VASC_REQUIRE(cdiv(total, 4) < (int64_t(1) << 31), "grid too large");
  hipLaunchKernelGGL(pair_innovation_kernel, dim3(cdiv(total, 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), pooled_v, kb, npairs, total, innovation);
  return check_launch("vasc_pair_innovation");
}

extern "C" int vasc_pooled_softmax(const uint16_t *pooled_q, const uint16_t *pooled_k, int64_t B, int64_t H,
                                   int64_t qb, int64_t kb, int64_t d, float scale, int32_t round_bf16, float *prob,
                                   void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == 64, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(pooled_q && pooled_k && prob && B > 0 && H > 0 && qb > 0 && kb > 0, "invalid arguments");
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(pooled_q) & 15) == 0 && (reinterpret_cast<uintptr_t>(pooled_k) & 15) == 0,
               "pooled inputs must be 16-byte aligned");
  VASC_REQUIRE(B * H < 65536, "grid too large");
  hipLaunchKernelGGL(pooled_softmax_kernel, dim3(cdiv(qb, 32), B * H), dim3(kSoftmaxWaves * 64), 0,
                     reinterpret_cast<hipStream_t>(stream), pooled_q, pooled_k, qb, kb, scale, round_bf16, prob);
  return check_launch("vasc_pooled_softmax");
}
