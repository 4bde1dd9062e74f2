// Kernel 1: block mean pooling of Q/K/V, pair innovation, pooled softmax.
//
// 1a (pool_qkv_kernel) is HBM-bound: each workgroup streams one 128-token
// span of Q, K and V (3 x 16 KB) with 16-byte coalesced loads, reduces the
// 8-lane groups that share a 16-byte column with DPP moves (no LDS traffic)
// and the four waves through LDS, and writes one pooled Q row, two pooled K
// rows and two
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

// kMax: block max of Q and K instead of the mean (predict_attention with
// pool_mode="max", F.max_pool1d with ceil_mode: a tail block takes the max of
// its real tokens). The max of bf16 values is exact; V is not pooled here.
template <bool kMax>
__global__ __launch_bounds__(256) void pool_qkv_kernel(const PoolParams p) {
  __shared__ float red[3][2][4][kHeadDim];
  __shared__ float pv[2][kHeadDim];
  const int64_t chunk = blockIdx.x;  // 128-token span
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  // lane bits 0-2: token within a group of 8, bits 3-5: 16-byte feature
  // chunk; a load instruction still covers 8 whole 128-byte rows, and the
  // token reduction stays inside DPP groups of 8 lanes
  const int t8 = lane & 7, dc = lane >> 3;

  // Issue all 12 row loads (3 tensors x 4 rows) before any reduction so each
  // thread keeps 192 bytes in flight.
  u32x4 raw[3][4];
#pragma unroll
  for (int X = 0; X < 3; ++X) {
    const uint16_t *src = p.x[X] ? p.x[X] + b * p.sb[X] + h * p.sh[X] + dc * 8 : nullptr;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t tok = chunk * 128 + 32 * u + 8 * w + t8;
      constexpr uint32_t kPad = kMax ? 0xff80ff80u : 0u;  // -inf pairs: missing tokens never win a max
      raw[X][u] = (src && tok < p.ntok[X]) ? *reinterpret_cast<const u32x4 *>(src + tok * p.st[X])
                                           : u32x4{kPad, kPad, kPad, kPad};
    }
  }
#pragma unroll
  for (int X = 0; X < 3; ++X) {
    if (p.x[X] == nullptr) continue;
    float acc[2][8];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[half][i] = kMax ? -INFINITY : 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(raw[X][u][i] << 16), hi = __uint_as_float(raw[X][u][i] & 0xffff0000u);
        if (kMax) {
          acc[u >> 1][2 * i] = fmaxf(acc[u >> 1][2 * i], lo);
          acc[u >> 1][2 * i + 1] = fmaxf(acc[u >> 1][2 * i + 1], hi);
        } else {
          acc[u >> 1][2 * i] += lo;
          acc[u >> 1][2 * i + 1] += hi;
        }
      }
    }
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[half][i] = kMax ? group8_max(acc[half][i]) : group8_sum(acc[half][i]);
    if (t8 == 0) {
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
      if (kMax)
        sum = fmaxf(fmaxf(fmaxf(red[0][0][0][d], red[0][0][1][d]), fmaxf(red[0][0][2][d], red[0][0][3][d])),
                    fmaxf(fmaxf(red[0][1][0][d], red[0][1][1][d]), fmaxf(red[0][1][2][d], red[0][1][3][d])));
      else
        sum = ((red[0][0][0][d] + red[0][0][1][d]) + (red[0][0][2][d] + red[0][0][3][d])) +
              ((red[0][1][0][d] + red[0][1][1][d]) + (red[0][1][2][d] + red[0][1][3][d]));
      blk = chunk;
      count = p.ntok[0] - chunk * 128;
      count = count > 128 ? 128 : count;
    } else {
      const int half = (slot - 1) & 1;
      if (kMax)
        sum = fmaxf(fmaxf(red[X][half][0][d], red[X][half][1][d]), fmaxf(red[X][half][2][d], red[X][half][3][d]));
      else
        sum = (red[X][half][0][d] + red[X][half][1][d]) + (red[X][half][2][d] + red[X][half][3][d]);
      blk = 2 * chunk + half;
      count = p.ntok[X] - blk * 64;
      count = count > 64 ? 64 : count;
    }
    if (count <= 0) continue;
    const uint16_t mean = f32_to_bf16(kMax ? sum : sum / static_cast<float>(count));  // a max is exact in bf16
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

constexpr float kLog2e = 1.44269504088896341f;

// How the fp32 MFMA dot turns into the logit; y = r * sc is the exp2
// argument (logit * log2 e), sc > 0.
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

__device__ __forceinline__ floatx16 tile_dots(const u32x4 (&a)[4], const u32x4 (&b)[4]) {
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma32(a[s], b[s], acc);
  return acc;
}

// Row (A-operand index) held by acc[r] of a lane in half hf of the 32x32
// MFMA output; the lane's column is its index mod 32.
__device__ __forceinline__ int acc_row(int r, int hf) { return 8 * (r >> 2) + 4 * hf + (r & 3); }

// (m, s) <- merge of two softmax states (max y, sum of exp2(y - max)).
__device__ __forceinline__ void merge_ms(float &m, float &s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = (m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f(m - mn)) +
      (m2 == -INFINITY ? 0.f : s2 * __builtin_amdgcn_exp2f(m2 - mn));
  m = mn;
}

// Both kernels work on blocks of 128 query rows x 256 keys of one head.
// Wave w of a block owns keys 32w .. 32w + 31 and keeps their pooled K rows
// in registers (the 32x32x16 A and B operands share one register layout:
// lane l holds row l % 32, dims 8 (l / 32) + 16 s .. + 7 in register s);
// the block's 128 pooled Q rows are staged in LDS with their 16-byte chunks
// XOR-swizzled by row, so the 32 rows a wave reads at once hit distinct
// banks. K and Q are read once per block.
constexpr int kBlockRows = 128, kBlockWaves = 8, kBlockKeys = 32 * kBlockWaves;

struct BlockParams {
  const uint16_t *pq, *pk;
  float2 *part;  // [B*H][nkb][qb] per-block row states (max y, sum exp2(y - max))
  float *prob;
  float *priority;  // optional: max(prob, 0) with NaN -> 0
  int64_t qb, kb, nrb, nkb, num_wg;
  float scale, sc;
};

struct BlockCoords {
  int64_t bh, R0, key0;  // head, first row, first key of the wave
  int rows, nkeys;       // valid rows of the block (1..128), valid keys of the wave (<= 0: none)
  int64_t kbk;
};

// Block of this workgroup; workgroups are ordered so that each XCD walks a
// contiguous run of (head, row block) pairs, key blocks innermost.
__device__ __forceinline__ BlockCoords block_coords(const BlockParams &p, int w) {
  BlockCoords c;
  const int64_t wg = xcd_remap(blockIdx.x, p.num_wg);
  c.kbk = wg % p.nkb;
  const int64_t rest = wg / p.nkb;
  c.bh = rest / p.nrb;
  c.R0 = (rest % p.nrb) * kBlockRows;
  c.rows = static_cast<int>(p.qb - c.R0 < kBlockRows ? p.qb - c.R0 : kBlockRows);
  c.key0 = c.kbk * kBlockKeys + 32 * w;
  const int64_t nk = p.kb - c.key0;
  c.nkeys = static_cast<int>(nk < 32 ? (nk > 0 ? nk : 0) : 32);
  return c;
}

// Stage the block's pooled Q rows (zero past qb) into qs (all threads).
__device__ __forceinline__ void stage_q(const BlockParams &p, const BlockCoords &c, uint16_t *qs, int tid) {
  for (int i = tid; i < kBlockRows * 8; i += kBlockWaves * 64) {
    const int row = i >> 3, ch = i & 7;
    u32x4 v = {0, 0, 0, 0};
    if (row < c.rows) v = *reinterpret_cast<const u32x4 *>(p.pq + (c.bh * p.qb + c.R0 + row) * kHeadDim + 8 * ch);
    *reinterpret_cast<u32x4 *>(qs + row * kHeadDim + 8 * (ch ^ (row & 7))) = v;
  }
}

// Operand registers of the wave's 32 keys (key clamped into [0, kb)).
__device__ __forceinline__ void load_key_tile(const BlockParams &p, const BlockCoords &c, int lr, int hf,
                                              u32x4 (&k)[4]) {
  const int64_t key = lr < c.nkeys ? c.key0 + lr : c.key0;
  const uint16_t *kr = p.pk + (c.bh * p.kb + key) * kHeadDim + 8 * hf;
#pragma unroll
  for (int s = 0; s < 4; ++s) k[s] = *reinterpret_cast<const u32x4 *>(kr + 16 * s);
}

// Operand registers of staged Q rows 32 j .. 32 j + 31.
__device__ __forceinline__ void read_q_tile(const uint16_t *qs, int j, int lr, int hf, u32x4 (&q)[4]) {
  const int row = 32 * j + lr;
#pragma unroll
  for (int s = 0; s < 4; ++s) q[s] = *reinterpret_cast<const u32x4 *>(qs + row * kHeadDim + 8 * ((2 * s + hf) ^ (row & 7)));
}

// Per-block row states. The wave computes S^T = K Q^T (lane = query row,
// its 16 accumulators = 16 of the wave's keys), takes the lane's max y and
// sum of exp2(y - max) over those keys, merges the two halves (the other 16
// keys) and then the 8 waves through LDS, and writes (max, sum) of every
// row over the block's 256 keys.
template <int kMode>
__global__ __launch_bounds__(kBlockWaves * 64) void pooled_stats_kernel(const BlockParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t qs[kBlockRows * kHeadDim];
  __shared__ float wm[kBlockWaves][kBlockRows], wsum[kBlockWaves][kBlockRows];
  const int tid = threadIdx.x, l = tid & 63, lr = l & 31, hf = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const BlockCoords c = block_coords(p, w);
  stage_q(p, c, qs, tid);
  u32x4 kt[4];
  if (c.nkeys > 0) load_key_tile(p, c, lr, hf, kt);
  __syncthreads();
  if (c.nkeys > 0) {
    for (int j = 0; j < kBlockRows / 32; ++j) {
      if (32 * j >= c.rows) break;
      u32x4 qt[4];
      read_q_tile(qs, j, lr, hf, qt);
      floatx16 acc = tile_dots(kt, qt);
      dots_to_r<kMode>(acc, p.scale);
      if (c.nkeys < 32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = acc_row(r, hf) < c.nkeys ? acc[r] : -INFINITY;
      }
      float mr = acc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mr = fmaxf(mr, acc[r]);
      float m = mr * p.sc, s = 0.f;
      if (m != -INFINITY) {
        float e[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(fmaf(acc[r], p.sc, -m));
#pragma unroll
        for (int r = 0; r < 16; r += 2) e[r] += e[r + 1];
#pragma unroll
        for (int r = 0; r < 16; r += 4) e[r] += e[r + 2];
        s = (e[0] + e[4]) + (e[8] + e[12]);
      }
      merge_ms(m, s, __shfl_xor(m, 32), __shfl_xor(s, 32));
      if (hf == 0) {
        wm[w][32 * j + lr] = m;
        wsum[w][32 * j + lr] = s;
      }
    }
  }
  __syncthreads();
  if (tid < c.rows) {
    const int nw = static_cast<int>((p.kb - c.kbk * kBlockKeys + 31) / 32);  // waves with keys
    float m = wm[0][tid], s = wsum[0][tid];
    for (int i = 1; i < (nw < kBlockWaves ? nw : kBlockWaves); ++i) merge_ms(m, s, wm[i][tid], wsum[i][tid]);
    p.part[(c.bh * p.nkb + c.kbk) * p.qb + c.R0 + tid] = float2{m, s};
  }
}

// Normalised probabilities: merges the row states of the nkb key blocks
// into (max, 1 / sum) per row, then wave w walks the block's four 32-row
// tiles with its keys' operand in registers and writes
// exp2(y - max) / sum; a store covers two rows of 32 consecutive keys.
template <int kMode>
__global__ __launch_bounds__(kBlockWaves * 64) void pooled_prob_kernel(const BlockParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t qs[kBlockRows * kHeadDim];
  __shared__ __attribute__((aligned(16))) float sgm[kBlockRows], sinv[kBlockRows];
  const int tid = threadIdx.x, l = tid & 63, lr = l & 31, hf = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const BlockCoords c = block_coords(p, w);
  stage_q(p, c, qs, tid);
  {
    // 4 threads per row, each merging every 4th key block's state
    const int row = tid >> 2, q4 = tid & 3;
    float m = -INFINITY, s = 0.f;
    if (row < c.rows) {
      const float2 *pr = p.part + c.bh * p.nkb * p.qb + c.R0 + row;
      for (int64_t i0 = q4; i0 < p.nkb; i0 += 16) {
        // the four loads are issued together, then merged
        float2 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = i0 + 4 * k < p.nkb ? pr[(i0 + 4 * k) * p.qb] : float2{-INFINITY, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) merge_ms(m, s, v[k].x, v[k].y);
      }
    }
    merge_ms(m, s, __shfl_xor(m, 1), __shfl_xor(s, 1));
    merge_ms(m, s, __shfl_xor(m, 2), __shfl_xor(s, 2));
    if (q4 == 0) {
      sgm[row] = m;
      sinv[row] = s > 0.f ? 1.f / s : 0.f;
    }
  }
  u32x4 kt[4];
  if (c.nkeys > 0) load_key_tile(p, c, lr, hf, kt);
  __syncthreads();
  if (c.nkeys <= 0) return;
  const bool full = c.nkeys == 32 && c.rows == kBlockRows;
  const int kb = static_cast<int>(p.kb);
  float *base = p.prob + (c.bh * p.qb + c.R0) * p.kb + c.key0;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      base, 0, static_cast<int>((static_cast<int64_t>(c.rows - 1) * p.kb + c.nkeys) * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t prio = __builtin_amdgcn_make_buffer_rsrc(
      p.priority ? p.priority + (base - p.prob) : base, 0,
      p.priority ? static_cast<int>((static_cast<int64_t>(c.rows - 1) * p.kb + c.nkeys) * 4) : 0, 0x00020000);
  uint32_t soff[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) soff[r] = static_cast<uint32_t>(acc_row(r, 0) * kb * 4);
  const bool kok = lr < c.nkeys;
  for (int j = 0; j < kBlockRows / 32; ++j) {
    if (32 * j >= c.rows) break;
    u32x4 qt[4];
    read_q_tile(qs, j, lr, hf, qt);
    floatx16 acc = tile_dots(qt, kt);  // lane = key, accumulators = rows
    dots_to_r<kMode>(acc, p.scale);
    float gm[16], inv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const floatx4 m4 = *reinterpret_cast<const floatx4 *>(sgm + 32 * j + 8 * g + 4 * hf);
      const floatx4 i4 = *reinterpret_cast<const floatx4 *>(sinv + 32 * j + 8 * g + 4 * hf);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gm[4 * g + e] = m4[e];
        inv[4 * g + e] = i4[e];
      }
    }
    const uint32_t voff = static_cast<uint32_t>(((32 * j + 4 * hf) * kb + lr) * 4);
    // row 32 j + acc_row(r, hf) < rows <=> acc_row(r, 0) < rlim
    const int rlim = c.rows - 32 * j - 4 * hf;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = __builtin_amdgcn_exp2f(fmaf(acc[r], p.sc, -gm[r])) * inv[r];
      // invalid lanes get a vector offset of 2^31, past the buffer's end
      // (below 2^31) with or without the scalar row offset: the store is dropped
      const bool ok = full || (kok && acc_row(r, 0) < rlim);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pr), rsrc, ok ? voff : 0x80000000u, soff[r], 0);
      // a null priority has a zero-size range: the store is dropped
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pr > 0.f ? pr : 0.f), prio, ok ? voff : 0x80000000u,
                                            soff[r], 0);
    }
  }
}

// One launch for rows of at most 256 kTiles keys: workgroup g takes the 32
// pooled query rows 32 (g % nrt) .. of head g / nrt against every key of the
// head. Wave w holds the key tiles w, w + 8, .. (32 keys each) as the
// accumulators of S = Q K^T (lane = key, accumulators = rows), so each logit
// is computed once and stays in registers: the row maxima are reduced across
// the 32 lanes of a half and then the eight waves through LDS, the row sums
// of exp2(y - max) likewise, and the normalised probabilities are written
// from the same registers (a store covers two rows of 32 consecutive keys).
// Needs no workspace.
template <int kMode, int kTiles>
__global__ __launch_bounds__(kBlockWaves * 64) void pooled_rows_kernel(const BlockParams p) {
  __shared__ float red[kBlockWaves][32];
  __shared__ __attribute__((aligned(16))) float rowv[32];
  const int tid = threadIdx.x, l = tid & 63, lr = l & 31, hf = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t wg = xcd_remap(blockIdx.x, p.num_wg);
  const int64_t bh = wg / p.nrb;
  const int64_t R0 = (wg % p.nrb) * 32;
  const int rows = static_cast<int>(p.qb - R0 < 32 ? p.qb - R0 : 32);
  const int kb = static_cast<int>(p.kb);
  u32x4 qt[4], kt[kTiles][4];
  {
    const uint16_t *qr = p.pq + (bh * p.qb + R0 + (lr < rows ? lr : 0)) * kHeadDim + 8 * hf;
#pragma unroll
    for (int s = 0; s < 4; ++s) qt[s] = *reinterpret_cast<const u32x4 *>(qr + 16 * s);
  }
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    const int key0 = 32 * (w + kBlockWaves * i);
    if (key0 >= kb) break;
    const int key = key0 + lr < kb ? key0 + lr : key0;
    const uint16_t *kr = p.pk + (bh * p.kb + key) * kHeadDim + 8 * hf;
#pragma unroll
    for (int s = 0; s < 4; ++s) kt[i][s] = *reinterpret_cast<const u32x4 *>(kr + 16 * s);
  }
  floatx16 acc[kTiles];
  float m[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) m[r] = -INFINITY;
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    const int key0 = 32 * (w + kBlockWaves * i);
    if (key0 < kb) {
      acc[i] = tile_dots(qt, kt[i]);
      dots_to_r<kMode>(acc[i], p.scale);
      if (key0 + lr >= kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = -INFINITY;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = fmaxf(m[r], acc[i][r]);
  }
#pragma unroll
  for (int off = 1; off < 32; off <<= 1)
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = fmaxf(m[r], xor_lane(m[r], off));
  if (lr == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[w][acc_row(r, hf)] = m[r];
  }
  __syncthreads();
  if (tid < 32) {
    float g = red[0][tid];
#pragma unroll
    for (int i = 1; i < kBlockWaves; ++i) g = fmaxf(g, red[i][tid]);
    rowv[tid] = g * p.sc;  // the row's largest exp2 argument
  }
  __syncthreads();
  float gm[16];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const floatx4 m4 = *reinterpret_cast<const floatx4 *>(rowv + 8 * g + 4 * hf);
#pragma unroll
    for (int e = 0; e < 4; ++e) gm[4 * g + e] = m4[e];
  }
  float sum[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sum[r] = 0.f;
#pragma unroll
  for (int i = 0; i < kTiles; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc[i][r] = __builtin_amdgcn_exp2f(fmaf(acc[i][r], p.sc, -gm[r]));
      sum[r] += acc[i][r];
    }
#pragma unroll
  for (int off = 1; off < 32; off <<= 1)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum[r] += xor_lane(sum[r], off);
  if (lr == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[w][acc_row(r, hf)] = sum[r];
  }
  __syncthreads();
  if (tid < 32) {
    float t = red[0][tid];
#pragma unroll
    for (int i = 1; i < kBlockWaves; ++i) t += red[i][tid];
    rowv[tid] = 1.f / t;
  }
  __syncthreads();
  float inv[16];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const floatx4 i4 = *reinterpret_cast<const floatx4 *>(rowv + 8 * g + 4 * hf);
#pragma unroll
    for (int e = 0; e < 4; ++e) inv[4 * g + e] = i4[e];
  }
  float *base = p.prob + (bh * p.qb + R0) * p.kb;
  const int bytes = rows * kb * 4;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t prio = __builtin_amdgcn_make_buffer_rsrc(
      p.priority ? p.priority + (bh * p.qb + R0) * p.kb : base, 0, p.priority ? bytes : 0, 0x00020000);
  const int rlim = rows - 4 * hf;  // row acc_row(r, hf) < rows <=> acc_row(r, 0) < rlim
#pragma unroll
  for (int i = 0; i < kTiles; ++i) {
    const int key0 = 32 * (w + kBlockWaves * i);
    if (key0 >= kb) break;
    const bool kok = key0 + lr < kb;
    const uint32_t voff = static_cast<uint32_t>(((4 * hf) * kb + key0 + lr) * 4);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = acc[i][r] * inv[r];
      // rows past qb and keys past kb: an offset of 2^31 lies past the range
      const uint32_t off = kok && acc_row(r, 0) < rlim ? voff : 0x80000000u;
      const uint32_t soff = static_cast<uint32_t>(acc_row(r, 0) * kb * 4);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pr), rsrc, off, soff, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(pr > 0.f ? pr : 0.f), prio, off, soff, 0);
    }
  }
}

// key tiles per wave of pooled_rows_kernel for kb keys (0: the two-kernel path)
constexpr int kRowTileSteps[] = {1, 2, 3, 5};
inline int row_tiles(int64_t kb) {
  for (int t : kRowTileSteps)
    if (kb <= 32 * kBlockWaves * t) return t;
  return 0;
}

}  // namespace
}  // namespace vasc

namespace vasc {
namespace {
int pool_impl(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const uint16_t *k,
                             int64_t k_sb, int64_t k_sh, int64_t k_st, const uint16_t *v, int64_t v_sb,
                             int64_t v_sh, int64_t v_st, int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d,
                             int64_t block_q, int64_t block_k, uint16_t *pooled_q, uint16_t *pooled_k,
                             uint16_t *pooled_v, float *innovation, void *stream, bool pool_max) {
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
  if (pool_max)
    hipLaunchKernelGGL(pool_qkv_kernel<true>, dim3(chunks, B * H), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       p);
  else
    hipLaunchKernelGGL(pool_qkv_kernel<false>, dim3(chunks, B * H), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), p);
  return check_launch(pool_max ? "vasc_pool_qk_max" : "vasc_pool_qkv");
}
}  // namespace
}  // namespace vasc

extern "C" int vasc_pool_qkv(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const uint16_t *k,
                             int64_t k_sb, int64_t k_sh, int64_t k_st, const uint16_t *v, int64_t v_sb,
                             int64_t v_sh, int64_t v_st, int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d,
                             int64_t block_q, int64_t block_k, uint16_t *pooled_q, uint16_t *pooled_k,
                             uint16_t *pooled_v, float *innovation, void *stream) {
  return vasc::pool_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, B, H, nq, nk, d, block_q,
                         block_k, pooled_q, pooled_k, pooled_v, innovation, stream, false);
}

extern "C" int vasc_pool_qk_max(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st, const uint16_t *k,
                                int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t B, int64_t H, int64_t nq,
                                int64_t nk, int64_t d, int64_t block_q, int64_t block_k, uint16_t *pooled_q,
                                uint16_t *pooled_k, void *stream) {
  return vasc::pool_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, nullptr, 0, 0, 8, B, H, nq, nk, d, block_q,
                         block_k, pooled_q, pooled_k, nullptr, nullptr, stream, true);
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

extern "C" int64_t vasc_pooled_softmax_workspace_size(int64_t B, int64_t H, int64_t qb, int64_t kb) {
  using namespace vasc;
  if (row_tiles(kb)) return 0;  // one launch, no row states
  return B > 0 && H > 0 && qb > 0 && kb > 0 ? B * H * cdiv(kb, kBlockKeys) * qb * 8 : 0;
}

extern "C" int vasc_pooled_softmax(const uint16_t *pooled_q, const uint16_t *pooled_k, int64_t B, int64_t H,
                                   int64_t qb, int64_t kb, int64_t d, float scale, int32_t round_bf16, float *prob,
                                   float *priority, void *workspace, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == 64, "head_dim %lld not built (built: 64)", (long long)d);
  const int tiles = row_tiles(kb);
  VASC_REQUIRE(pooled_q && pooled_k && prob && (workspace || tiles) && B > 0 && H > 0 && qb > 0 && kb > 0,
               "invalid arguments (pooled_q, pooled_k, prob and, for kb > %d, workspace are required)",
               32 * kBlockWaves * kRowTileSteps[3]);
  VASC_REQUIRE(std::isfinite(scale) && scale > 0.f, "scale must be finite and positive");
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(pooled_q) & 15) == 0 && (reinterpret_cast<uintptr_t>(pooled_k) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(workspace) & 7) == 0,
               "pooled inputs must be 16-byte aligned, the workspace 8-byte aligned");
  // a probability block (128 rows x kb fp32) is addressed with 32-bit offsets
  VASC_REQUIRE(kb < (int64_t(1) << 22), "kb %lld not below 2^22", (long long)kb);
  BlockParams p;
  p.pq = pooled_q;
  p.pk = pooled_k;
  p.part = static_cast<float2 *>(workspace);
  p.prob = prob;
  p.priority = priority;
  p.qb = qb;
  p.kb = kb;
  int e = 0;
  const bool pow2 = std::frexp(scale, &e) == 0.5f;
  const int mode = !round_bf16 ? kFp32 : pow2 ? kRoundPow2 : kRoundAny;
  p.scale = scale;
  p.sc = mode == kRoundAny ? kLog2e : scale * kLog2e;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (tiles) {
    p.nrb = cdiv(qb, 32);
    p.nkb = 1;
    p.num_wg = p.nrb * B * H;
    VASC_REQUIRE(p.num_wg < (int64_t(1) << 31), "grid too large");
    using Kern = void (*)(BlockParams);
    static constexpr Kern kRows[3][4] = {
        {pooled_rows_kernel<kRoundPow2, 1>, pooled_rows_kernel<kRoundPow2, 2>, pooled_rows_kernel<kRoundPow2, 3>,
         pooled_rows_kernel<kRoundPow2, 5>},
        {pooled_rows_kernel<kRoundAny, 1>, pooled_rows_kernel<kRoundAny, 2>, pooled_rows_kernel<kRoundAny, 3>,
         pooled_rows_kernel<kRoundAny, 5>},
        {pooled_rows_kernel<kFp32, 1>, pooled_rows_kernel<kFp32, 2>, pooled_rows_kernel<kFp32, 3>,
         pooled_rows_kernel<kFp32, 5>}};
    const int ti = tiles == 1 ? 0 : tiles == 2 ? 1 : tiles == 3 ? 2 : 3;
    hipLaunchKernelGGL(kRows[mode][ti], dim3(p.num_wg), dim3(kBlockWaves * 64), 0, st, p);
    return check_launch("vasc_pooled_softmax");
  }
  p.nrb = cdiv(qb, kBlockRows);
  p.nkb = cdiv(kb, kBlockKeys);
  p.num_wg = p.nrb * p.nkb * B * H;
  VASC_REQUIRE(p.num_wg < (int64_t(1) << 31), "grid too large");
  auto ks = mode == kRoundPow2 ? pooled_stats_kernel<kRoundPow2>
            : mode == kRoundAny ? pooled_stats_kernel<kRoundAny>
                                : pooled_stats_kernel<kFp32>;
  hipLaunchKernelGGL(ks, dim3(p.num_wg), dim3(kBlockWaves * 64), 0, st, p);
  auto kp = mode == kRoundPow2 ? pooled_prob_kernel<kRoundPow2>
            : mode == kRoundAny ? pooled_prob_kernel<kRoundAny>
                                : pooled_prob_kernel<kFp32>;
  hipLaunchKernelGGL(kp, dim3(p.num_wg), dim3(kBlockWaves * 64), 0, st, p);
  return check_launch("vasc_pooled_softmax");
}

