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
// 1b (pooled_softmax_kernel) computes the pooled logits on MFMA in the
// standard output layout (a wave's store writes two rows of 32 consecutive
// keys) in two passes: per-row sums of exp2(logit * log2 e), then the
// normalised write, recomputing the logits. Rows whose sum leaves a safe
// range are redone with an online (max, sum) pass. Its cost is the fp32
// write of the [Qb, Kb] probability matrix.
//
// Reference: predict_attention (attention.py:31-104),
// _mean_pool_contiguous_value_blocks (sparse_wrapper.py:2839-2861),
// pair innovation (sparse_wrapper.py:3733-3740).
#include <cmath>
#include <type_traits>

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

constexpr int kSoftmaxWaves = 8;  // key tiles of one 32-row strip spread over 8 waves
constexpr float kLog2e = 1.44269504088896341f;
// A row whose sum of exp2(y) over its keys lies in [kSumLow, kSumHigh] took
// no overflowed term and keeps full relative precision, so the fast pass
// (no running max) is exact enough; any other row sends the strip through
// the online (max, sum) pass.
constexpr float kSumHigh = 0x1p100f, kSumLow = 0x1p-60f;

// How the fp32 MFMA dot turns into the logit; y = r * sc is the exp2
// argument (logit * log2 e).
enum LogitMode : int {
  kRoundPow2 = 0,  // bf16(bf16(dot) * scale) with scale a power of two: = bf16(dot) * scale exactly
  kRoundAny = 1,   // bf16(bf16(dot) * scale)
  kFp32 = 2,       // dot * scale
};

template <int kMode>
__device__ __forceinline__ void dots_to_r(floatx16 &acc, float scale) {
  if constexpr (kMode != kFp32) {
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      uint32_t h = pack_bf16x2(acc[i], acc[i + 1]);
      float a = __uint_as_float(h << 16), b = __uint_as_float(h & 0xffff0000u);
      if constexpr (kMode == kRoundAny) {
        h = pack_bf16x2(a * scale, b * scale);
        a = __uint_as_float(h << 16);
        b = __uint_as_float(h & 0xffff0000u);
      }
      acc[i] = a;
      acc[i + 1] = b;
    }
  }
}

// B operand of the 32-key tile whose first key is key0 (lane: key
// key0 + lr, dims 16s + 8hf .. +7), key clamped into [0, kb).
__device__ __forceinline__ void load_keys(const uint16_t *kbase, int64_t key, int hf, u32x4 (&b)[4]) {
  const uint16_t *kr = kbase + key * kHeadDim + 8 * hf;
#pragma unroll
  for (int s = 0; s < 4; ++s) b[s] = *reinterpret_cast<const u32x4 *>(kr + 16 * s);
}

__device__ __forceinline__ floatx16 tile_dots(const u32x4 (&qa)[4], const u32x4 (&b)[4]) {
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma32(qa[s], b[s], acc);
  return acc;
}

// Strip row held by acc[r] of a lane in half hf (standard 32x32 MFMA output).
__device__ __forceinline__ int acc_row(int r, int hf) { return 8 * (r >> 2) + 4 * hf + (r & 3); }

struct SoftmaxStrip {
  const uint16_t *kbase;
  float *out;  // row0 of the strip
  int64_t kb, nfull, rows;  // keys, full 32-key tiles, valid rows of the strip (1..32)
  float scale, sc;
  int w, lr, hf;
};

// exp2(y) of one tile into the lane's 16 row sums (fast pass).
template <int kMode, bool kMasked>
__device__ __forceinline__ void sum_tile(const SoftmaxStrip &st, const u32x4 (&qa)[4], const u32x4 (&b)[4], int64_t t,
                                         float (&sum)[16]) {
  floatx16 acc = tile_dots(qa, b);
  dots_to_r<kMode>(acc, st.scale);
  const bool ok = !kMasked || 32 * t + st.lr < st.kb;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float e = __builtin_amdgcn_exp2f(acc[r] * st.sc);
    sum[r] += ok ? e : 0.f;
  }
}

// Online (max, sum) of y over one tile (exact pass).
template <int kMode, bool kMasked>
__device__ __forceinline__ void online_tile(const SoftmaxStrip &st, const u32x4 (&qa)[4], const u32x4 (&b)[4],
                                            int64_t t, float (&m)[16], float (&sum)[16]) {
  floatx16 acc = tile_dots(qa, b);
  dots_to_r<kMode>(acc, st.scale);
  const bool ok = !kMasked || 32 * t + st.lr < st.kb;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const float y = acc[r] * st.sc;
    const float d = y - m[r];
    const bool up = d > 0.f;  // false for NaN
    const float e = __builtin_amdgcn_exp2f(up ? -d : d);
    const float s_up = m[r] == -INFINITY ? 1.f : fmaf(sum[r], e, 1.f);
    if (ok) {
      sum[r] = up ? s_up : sum[r] + e;
      m[r] = up ? y : m[r];
    }
  }
}

// Normalised probabilities of one tile: exp2(y - gm) * inv.
template <int kMode, bool kExact, bool kMasked>
__device__ __forceinline__ void store_tile(const SoftmaxStrip &st, const u32x4 (&qa)[4], const u32x4 (&b)[4],
                                           int64_t t, const float (&gm)[16], const float (&inv)[16],
                                           __amdgpu_buffer_rsrc_t rsrc, const uint32_t (&soff)[16]) {
  floatx16 acc = tile_dots(qa, b);
  dots_to_r<kMode>(acc, st.scale);
  if (!kMasked) {
    const uint32_t voff = static_cast<uint32_t>((4 * st.hf * st.kb + 32 * t + st.lr) * 4);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float y = kExact ? acc[r] * st.sc - gm[r] : acc[r] * st.sc;  // y rounded as in pass 1
      const float pr = __builtin_amdgcn_exp2f(y) * inv[r];
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pr), rsrc, voff, soff[r], 0);
    }
  } else {
    // Invalid lanes get a vector offset of 2^31, past the buffer's end
    // (num_records < 2^31) whether or not the scalar row offset is added
    // (it is below 2^31): the store is dropped.
    const int64_t key = 32 * t + st.lr;
    const uint32_t voff = static_cast<uint32_t>((4 * st.hf * st.kb + key) * 4);
    const bool kok = key < st.kb;
    const int rlim = static_cast<int>(st.rows) - 4 * st.hf;  // acc_row(r, hf) < rows <=> acc_row(r, 0) < rlim
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float y = kExact ? acc[r] * st.sc - gm[r] : acc[r] * st.sc;  // y rounded as in pass 1
      const bool ok = kok && acc_row(r, 0) < rlim;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(__builtin_amdgcn_exp2f(y) * inv[r]), rsrc,
                                            ok ? voff : 0x80000000u, soff[r], 0);
    }
  }
}

template <bool kMasked>
using Masked = std::integral_constant<bool, kMasked>;

// Calls f(keys, t, Masked<...>) for the wave's tiles t = w, w + 8, ... in
// order, the last (partial) tile masked. The B operand of the next tile is
// loaded into the other register set before the current tile's work (no
// copies, so the load stays in flight during that work).
template <class F>
__device__ __forceinline__ void walk_tiles(const SoftmaxStrip &st, int64_t first_key, F &&f) {
  constexpr int kW = kSoftmaxWaves;
  u32x4 k0[4], k1[4];
  int64_t t = st.w;
  load_keys(st.kbase, first_key, st.hf, k0);
  // Pairs of tiles with no exit between them, so neither load can be sunk
  // next to its use.
  while (t + kW < st.nfull) {
    load_keys(st.kbase, 32 * (t + kW) + st.lr, st.hf, k1);
    __builtin_amdgcn_sched_barrier(0);
    f(k0, t, Masked<false>{});
    __builtin_amdgcn_sched_barrier(0);
    const int64_t n0 = t + 2 * kW < st.nfull ? t + 2 * kW : t + kW;
    load_keys(st.kbase, 32 * n0 + st.lr, st.hf, k0);
    __builtin_amdgcn_sched_barrier(0);
    f(k1, t + kW, Masked<false>{});
    __builtin_amdgcn_sched_barrier(0);
    t += 2 * kW;
  }
  if (t < st.nfull) {
    f(k0, t, Masked<false>{});
    t += kW;
  }
  if (st.nfull * 32 < st.kb && t == st.nfull) {
    const int64_t key = 32 * t + st.lr;
    load_keys(st.kbase, key < st.kb ? key : st.kb - 1, st.hf, k0);
    f(k0, t, Masked<true>{});
  }
}

// (m, s) <- merge of two online-softmax states (max, sum of exp2(y - max)).
__device__ __forceinline__ void merge_ms(float &m, float &s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = (m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f(m - mn)) +
      (m2 == -INFINITY ? 0.f : s2 * __builtin_amdgcn_exp2f(m2 - mn));
  m = mn;
}

// Pass 2 of a wave: its tiles' normalised probabilities. kExact applies the
// per-row max (online pass) and the row mask of a partial strip.
template <int kMode, bool kExact>
__device__ __forceinline__ void write_pass(const SoftmaxStrip &st, const u32x4 (&qa)[4], int64_t first_key,
                                           const float *fin_m, const float *fin_inv) {
  float gm[16], inv[16];
  uint32_t soff[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    gm[r] = kExact ? fin_m[acc_row(r, st.hf)] : 0.f;
    inv[r] = fin_inv[acc_row(r, st.hf)];
    soff[r] = static_cast<uint32_t>(acc_row(r, 0) * st.kb * 4);
  }
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(st.out, 0, static_cast<int>(st.rows * st.kb * 4), 0x00020000);
  walk_tiles(st, first_key, [&](const u32x4(&b)[4], int64_t t, auto masked) {
    // the exact variant (rare: extreme rows or the partial last strip)
    // always takes the masked store
    constexpr bool kM = decltype(masked)::value || kExact;
    store_tile<kMode, kExact, kM>(st, qa, b, t, gm, inv, rsrc, soff);
  });
}

// One workgroup per (32-row strip, head); the workgroup walks the strip's
// key tiles twice, wave w taking tiles w, w + 8, ...:
//   pass 1 sums exp2(y) per row with no running max; rows whose sum falls
//          outside [kSumLow, kSumHigh] send the whole strip through an exact
//          online (max, sum) pass instead;
//   pass 2 recomputes each tile and writes exp2(y - max) / sum, a wave's
//          store covering two rows of 32 consecutive keys.
// Workgroups are ordered so that each XCD walks the strips of a contiguous
// run of heads (the heads' pooled K stays in that XCD's L2).
template <int kMode>
__global__ __launch_bounds__(kSoftmaxWaves * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void pooled_softmax_kernel(const uint16_t *__restrict__ pq,
                                                                           const uint16_t *__restrict__ pk,
                                                                           int64_t qb, int64_t kb, int64_t nstrip,
                                                                           int64_t num_wg, float scale,
                                                                           float *__restrict__ prob) {
  __shared__ float part[kSoftmaxWaves][32][32];
  __shared__ float sm_m[kSoftmaxWaves][32], sm_s[kSoftmaxWaves][32];
  __shared__ float fin_m[32], fin_inv[32];
  __shared__ int slow_flag;
  const int64_t wg = xcd_remap(blockIdx.x, num_wg);
  const int64_t bh = wg / nstrip, row0 = (wg % nstrip) * 32;
  const int tid = threadIdx.x, l = tid & 63;
  SoftmaxStrip st;
  st.lr = l & 31;
  st.hf = l >> 5;
  st.w = __builtin_amdgcn_readfirstlane(tid >> 6);
  st.kb = kb;
  st.nfull = kb / 32;
  st.rows = qb - row0 < 32 ? qb - row0 : 32;
  st.scale = scale;
  st.sc = kMode == kRoundAny ? kLog2e : scale * kLog2e;
  st.kbase = pk + bh * kb * kHeadDim;
  st.out = prob + (bh * qb + row0) * kb;
  if (tid == 0) slow_flag = 0;
  // A operand: lane holds query row row0 + lr, dims 16s + 8hf .. +7.
  u32x4 qa[4];
  {
    const bool qok = st.lr < st.rows;
    const uint16_t *qr = pq + (bh * qb + row0 + (qok ? st.lr : 0)) * kHeadDim + 8 * st.hf;
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = qok ? *reinterpret_cast<const u32x4 *>(qr + 16 * s) : u32x4{0, 0, 0, 0};
  }
  const bool tail = st.nfull * 32 < kb;
  // first key the wave loads (in bounds even when it has no full tile)
  int64_t first_key = 32 * (st.w < st.nfull ? st.w : st.nfull - 1) + st.lr;
  if (first_key < 0 || first_key >= kb) first_key = kb - 1;

  // ---- pass 1 (fast): per-lane row sums of exp2(y)
  float sum[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sum[r] = 0.f;
  walk_tiles(st, first_key, [&](const u32x4(&b)[4], int64_t t, auto masked) {
    sum_tile<kMode, decltype(masked)::value>(st, qa, b, t, sum);
  });
#pragma unroll
  for (int r = 0; r < 16; ++r) part[st.w][acc_row(r, st.hf)][st.lr] = sum[r];
  __syncthreads();
  {
    // 16 threads per row: each adds 16 partials, then a 16-lane reduction.
    const int row = tid >> 4, j = tid & 15;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kSoftmaxWaves; ++w) v += part[w][row][j] + part[w][row][j + 16];
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, 16);
    if (j == 0) {
      fin_m[row] = 0.f;
      fin_inv[row] = 1.f / v;
      if (row < st.rows && !(v >= kSumLow && v <= kSumHigh)) slow_flag = 1;
    }
  }
  __syncthreads();
  const bool exact = slow_flag != 0;

  if (exact) {
    // ---- pass 1 (exact): online (max, sum) per lane and row
    float m[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      m[r] = -INFINITY;
      sum[r] = 0.f;
    }
    walk_tiles(st, first_key, [&](const u32x4(&b)[4], int64_t t, auto masked) {
      online_tile<kMode, decltype(masked)::value>(st, qa, b, t, m, sum);
    });
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) merge_ms(m[r], sum[r], __shfl_xor(m[r], o), __shfl_xor(sum[r], o));
    }
    if (st.lr == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sm_m[st.w][acc_row(r, st.hf)] = m[r];
        sm_s[st.w][acc_row(r, st.hf)] = sum[r];
      }
    }
    __syncthreads();
    if (tid < 32) {
      float gm = sm_m[0][tid], gs = sm_s[0][tid];
#pragma unroll
      for (int i = 1; i < kSoftmaxWaves; ++i) merge_ms(gm, gs, sm_m[i][tid], sm_s[i][tid]);
      fin_m[tid] = gm;
      fin_inv[tid] = gs > 0.f ? 1.f / gs : 0.f;
    }
    __syncthreads();
  }

  // ---- pass 2: normalised write
  if (exact || st.rows < 32)
    write_pass<kMode, true>(st, qa, first_key, fin_m, fin_inv);
  else
    write_pass<kMode, false>(st, qa, first_key, fin_m, fin_inv);
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
  // one strip's output (32 rows x kb fp32) is addressed with 32-bit offsets
  VASC_REQUIRE(kb < (int64_t(1) << 24), "kb %lld not below 2^24", (long long)kb);
  const int64_t nstrip = cdiv(qb, 32), num_wg = nstrip * B * H;
  VASC_REQUIRE(num_wg < (int64_t(1) << 31), "grid too large");
  int e = 0;
  const bool pow2 = std::isfinite(scale) && scale != 0.f && std::frexp(scale, &e) == 0.5f;
  const int mode = !round_bf16 ? kFp32 : pow2 ? kRoundPow2 : kRoundAny;
  auto kern = mode == kRoundPow2 ? pooled_softmax_kernel<kRoundPow2>
              : mode == kRoundAny ? pooled_softmax_kernel<kRoundAny>
                                  : pooled_softmax_kernel<kFp32>;
  hipLaunchKernelGGL(kern, dim3(num_wg), dim3(kSoftmaxWaves * 64), 0, reinterpret_cast<hipStream_t>(stream), pooled_q,
                     pooled_k, qb, kb, nstrip, num_wg, scale, prob);
  return check_launch("vasc_pooled_softmax");
}

