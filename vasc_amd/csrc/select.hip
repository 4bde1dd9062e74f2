// Kernel 2: block selection (Top-K and VASC value-risk pair debt) writing
// ascending block-index lists, with VASC's cross-layer ledger.
//
// Reference: get_block_mask (sparse_wrapper.py:1199-1268),
// get_cosa_value_risk_pair_debt_mask (sparse_wrapper.py:3632-4098) in the
// release configuration, _project_conservative_capped_mass (1755-1769),
// _reduce_qk_indices_to_pair (2922-2980), block_map_lut_triton
// (ZIP:spas_sage_attn/utils.py:54-87).
//
// Bit-exactness contract: every float32 operation below is rounded on its
// own (contraction is off for this file) and every sum uses one of the
// canonical float64 orders shared with the CPU oracle:
//   wave sum  lane j adds elements j, j+64, ... in order, then an xor
//             butterfly over offsets 32..1;
//   chunked   sequential sums of consecutive 32-row chunks, then a
//             sequential sum of the chunk partials (the arrival mean);
//   global    wave sum per head, then sequential over heads (the gate).
// Selection keeps the c largest priorities, ties to the lower block index.
//
// Launches (VASC mode), each reading the fp32 score matrix once:
//   arrival  one workgroup per (32-row chunk, head), one wave per row: the
//            row arrives in registers (K <= 4096; lane j holds elements
//            j + 64 m, the canonical lane order) or in LDS by DMA (larger
//            K); risk total, conservative arrival and pair reductions, and
//            the chunk's float64 column partials of the pair arrival
//            accumulated in row order;
//   head     per head: ledger settlement, arrival mean, pair capacity,
//            admitted debt, the head's partials of the global gate;
//   select   one row per wave (K <= 1024) or per workgroup, the row in
//            registers: priorities as order-preserving keys, a sampled
//            histogram bracketing the c-th largest, the exact threshold
//            among the bracketed candidates, compaction to the ascending
//            list staged in LDS, pair counts;
//   service  QK-admission service from the pair counts.
// Top-K mode runs the select launch alone.
#pragma clang fp contract(off)

#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"

#include <rocprim/block/block_radix_sort.hpp>

namespace vasc {
namespace {

constexpr float kFltMax = 3.402823466e38f;
constexpr float kFltMin = 1.175494351e-38f;
constexpr int kChunk = 32;       // rows per partial of the arrival mean
constexpr int kWaves = 4;        // waves per workgroup (both row kernels)
constexpr int kMaxPairsPerThread = 16;  // arrival column partials per thread (P <= 16 * threads)

__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (x == 0.f) u = 0u;
  if (x != x) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float clean_score(float s) {
  if (s != s) return 0.f;
  if (!(s > 0.f)) return 0.f;
  if (s == INFINITY) return kFltMax;
  return s;
}

__device__ __forceinline__ float clamp01(float x) { return x < 0.f ? 0.f : (x > 1.f ? 1.f : x); }
__device__ __forceinline__ float clamp_min0(float x) { return x > 0.f ? x : (x != x ? x : 0.f); }
// torch clamp_min(x, FLT_MIN): NaN propagates.
__device__ __forceinline__ float floor_tiny(float x) { return x < kFltMin ? kFltMin : x; }

__device__ __forceinline__ void wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

struct SelectParams {
  const float *score;
  const float *innovation;
  int64_t BH, Q, K, P;
  int32_t mode, topk, force_last, max_capacity, sink;
  const int32_t *row_cap;
  const uint8_t *protected_mask;
  const float *debt_in, *pending, *prev_service;
  float *debt_out, *arrival_out, *service_out;
  int32_t *gate_out;
  float *priority_out;
  uint8_t *mask_out;
  int32_t *index_out;
  int64_t width;
  int32_t *count_out;
  // workspace
  float *total, *rowpair, *adm;
  float2 *ia;  // (innovation, admitted debt) per pair, for the select pass
  double *part, *gate_part;
  int32_t *cap, *counts;
  int32_t *flags;  // per row: the select pass may take the fast path (register-row kernels)
  int64_t nchunks;
};

// ------------------------------------------------------------- cdf counts
// get_block_mask's cdf branch (sparse_wrapper.py:1238-1254) and the fill
// rule (ZIP:spas_sage_attn/utils.py:289). One workgroup per row: the row's
// order keys are sorted descending in LDS (bitonic; padding keys 0 sort
// last), then one lane walks the sorted values with a strictly sequential
// float32 running sum and counts the prefix that stays <= T_h. The count is
// raised to min_count (the ratio budget when both are given) and a count of
// 0 becomes 1. base_out (optional) adds the forced mixed tail: one more block
// when at least `count` other blocks beat the last one (greater key, or an
// equal key at a lower index), i.e. when the last block is not among the
// first `count` of the row.
__device__ __forceinline__ float key_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// The cdf count of one row from its keys sorted descending in LDS (a
// multiple of 64 of them): the length of the longest prefix whose strictly
// sequential float32 running sum stays <= T. The running sum is one chain
// of adds (the prefix sums fl(S + x) of the sorted values, 64 per batch of
// 16 LDS reads in flight); whether the prefix still holds is a second
// chain beside it (a prefix that once exceeds T ends, whatever follows).
// The LDS offset goes through an opaque VGPR: otherwise the compiler treats
// the single walking lane's values as uniform and moves them through SGPRs
// (readfirstlane and scalar ops between the adds, slower than the chain).
__device__ __forceinline__ int cdf_walk(const uint4 *k4, int K, float T) {
  float acc = 0.f;
  int n = 0;
  bool go = true;
  int z = 0;
  asm volatile("" : "+v"(z));
  for (int b = 0; go && 64 * b < K; ++b) {
    uint4 q[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] = k4[16 * b + j + z];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t kq[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // a padding key (0, past the row end) reads as NaN and ends the prefix
        acc = acc + key_value(kq[e]);
        go = go && acc <= T;
        n += go ? 1 : 0;
      }
    }
  }
  return n;
}

__global__ __launch_bounds__(256) void cdf_count_kernel(const float *score, int64_t H, int64_t Q, int K, int n2,
                                                        const float *thr, int32_t min_count, int32_t force_last,
                                                        int32_t *count_out, int32_t *base_out) {
  extern __shared__ __attribute__((aligned(16))) uint32_t ckeys[];  // [n2], read 16 bytes at a time
  __shared__ int sbeat;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const float *srow = score + row * K;
  const uint32_t last = order_key(srow[K - 1]);
  if (tid == 0) sbeat = 0;
  __syncthreads();
  int beat = 0;
  for (int k = tid; k < n2; k += 256) {
    const uint32_t kk = k < K ? order_key(srow[k]) : 0u;
    ckeys[k] = kk;
    beat += k < K - 1 && kk >= last;
  }
  if (force_last && base_out) atomicAdd(&sbeat, beat);
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int t = tid; t < (n2 >> 1); t += 256) {
        const int i = ((t & ~(stride - 1)) << 1) | (t & (stride - 1)), j = i + stride;  // stride: a power of two
        const uint32_t a = ckeys[i], b = ckeys[j];
        const bool desc = (i & size) == 0;
        if (desc ? a < b : a > b) {
          ckeys[i] = b;
          ckeys[j] = a;
        }
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    int n = cdf_walk(reinterpret_cast<const uint4 *>(ckeys), K, thr[(row / Q) % H]);
    n = n > min_count ? n : min_count;
    n = n == 0 ? 1 : (n > K ? K : n);
    count_out[row] = n;
    if (base_out) base_out[row] = n + ((force_last && n < K && sbeat >= n) ? 1 : 0);
  }
}

// The same count with the row sorted by rocPRIM's LDS block radix sort (256
// threads, kItems keys each; 8-bit digits, four passes over 32-bit keys)
// instead of the bitonic network, which costs O(K log^2 K) compare-exchanges
// with a barrier per stage. Keys load lane-strided (coalesced), padding keys
// 0 sort last; after the descending sort thread t holds ranks
// [kItems t, kItems t + kItems), which it writes back to LDS for the same
// sequential walk.
template <int kItems>
__global__ __launch_bounds__(256) void cdf_count_radix_kernel(const float *score, int64_t H, int64_t Q, int K,
                                                              const float *thr, int32_t min_count,
                                                              int32_t force_last, int32_t *count_out,
                                                              int32_t *base_out) {
  using Sort = rocprim::block_radix_sort<uint32_t, 256, kItems>;
  __shared__ union {
    typename Sort::storage_type sort;
    float4 vals4[64 * kItems];  // the sorted values, then their prefix sums
  } sm;
  __shared__ int sbeat, sfail, swalked;
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const float *srow = score + row * K;
  const uint32_t last = order_key(srow[K - 1]);
  if (tid == 0) {
    sbeat = 0;
    sfail = K;
  }
  uint32_t key[kItems];
  int beat = 0;
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int k = tid + 256 * i;
    key[i] = k < K ? order_key(srow[k]) : 0u;
    beat += k < K - 1 && key[i] >= last;
  }
  __syncthreads();
  if (force_last && base_out) atomicAdd(&sbeat, beat);
  Sort().sort_desc(key, sm.sort);
  __syncthreads();  // the sort's storage is reused for the sorted values
  float *vals = reinterpret_cast<float *>(sm.vals4);
#pragma unroll
  for (int i = 0; i < kItems; ++i) vals[kItems * tid + i] = key_value(key[i]);  // padding: NaN
  __syncthreads();
  const float T = thr[(row / Q) % H];
  if (tid == 0) {
    // the running sum alone is serial: prefix sums written in place, 64 per
    // batch (16 LDS reads in flight), until a batch ends above T (or NaN)
    int z = 0;
    asm volatile("" : "+v"(z));  // keeps the walk in VGPRs (see cdf_walk)
    float acc = 0.f;
    int b = 0;
    for (; 64 * b < K; ++b) {
      float4 q[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) q[j] = sm.vals4[16 * b + j + z];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        acc += q[j].x;
        q[j].x = acc;
        acc += q[j].y;
        q[j].y = acc;
        acc += q[j].z;
        q[j].z = acc;
        acc += q[j].w;
        q[j].w = acc;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) sm.vals4[16 * b + j + z] = q[j];
      if (!(acc <= T)) {
        ++b;
        break;
      }
    }
    swalked = 64 * b;
  }
  __syncthreads();
  // the prefix ends at the first sum that is not <= T (every later one is
  // past the prefix whatever its value)
  const int walked = swalked;
  int fail = K;
  for (int i = tid; i < walked; i += 256)
    if (!(vals[i] <= T)) fail = i < fail ? i : fail;
  if (fail < K) atomicMin(&sfail, fail);
  __syncthreads();
  if (tid == 0) {
    int n = sfail;
    n = n > min_count ? n : min_count;
    n = n == 0 ? 1 : (n > K ? K : n);
    count_out[row] = n;
    if (base_out) base_out[row] = n + ((force_last && n < K && sbeat >= n) ? 1 : 0);
  }
}

// ------------------------------------------------------------------ settle
// Settled debt of one ledger entry (sparse_wrapper.py:3793-3832).
__device__ __forceinline__ float settle_one(const SelectParams &p, int64_t i, float *refl, float *sig) {
  const float d0 = p.debt_in ? clamp_min0(p.debt_in[i]) : 0.f;
  if (!p.pending) {
    *refl = 0.f;
    *sig = 0.f;
    return d0;
  }
  *sig = p.prev_service ? p.prev_service[i] : 0.f;
  const float u = (d0 + p.pending[i]) - *sig;
  *refl = clamp_min0(-u);
  return clamp_min0(u);
}

// Lane k's value of v (k uniform).
__device__ __forceinline__ double read_lane(double v, int k) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b), k));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(b >> 32), k));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Settlement of eight pairs per thread, j = j0 + kStride u (u < 8): settled
// debt, reflection and consumed service. With all three ledger inputs present
// the loads are unconditional (indices clamped into the head, results past P
// unused), so all 24 are in flight together; otherwise settle_one per pair.
constexpr int kSettleBatch = 8;
template <int kStride>
__device__ __forceinline__ void settle_batch(const SelectParams &p, int64_t bh, int64_t j0, float (&d)[kSettleBatch],
                                             float (&refl)[kSettleBatch], float (&sig)[kSettleBatch]) {
  if (p.debt_in && p.pending && p.prev_service) {
    float a[kSettleBatch], b[kSettleBatch], c[kSettleBatch];
#pragma unroll
    for (int u = 0; u < kSettleBatch; ++u) {
      const int64_t j = j0 + kStride * u < p.P ? j0 + kStride * u : p.P - 1;
      a[u] = p.debt_in[bh * p.P + j];
      b[u] = p.pending[bh * p.P + j];
      c[u] = p.prev_service[bh * p.P + j];
    }
#pragma unroll
    for (int u = 0; u < kSettleBatch; ++u) {
      const float x = (clamp_min0(a[u]) + b[u]) - c[u];
      sig[u] = c[u];
      refl[u] = clamp_min0(-x);
      d[u] = clamp_min0(x);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kSettleBatch; ++u) {
      const int64_t j = j0 + kStride * u;
      d[u] = refl[u] = sig[u] = 0.f;
      if (j < p.P) d[u] = settle_one(p, bh * p.P + j, &refl[u], &sig[u]);
    }
  }
}

// Pair capacity of a head (sparse_wrapper.py:3788-3791): the mean of the
// rows' pair-arrival sums, a wave sum over the rows (loads 16 rows per lane
// at a time, their sum in order). One wave; every lane returns it.
__device__ __forceinline__ float pair_capacity(const SelectParams &p, int64_t bh, int lane) {
  double acc = 0.0;
  for (int64_t q0 = lane; q0 < p.Q; q0 += 64 * 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = p.rowpair[bh * p.Q + (q0 + 64 * u < p.Q ? q0 + 64 * u : p.Q - 1)];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (q0 + 64 * u < p.Q) acc = acc + static_cast<double>(v[u]);
  }
  return static_cast<float>(wave_butterfly(acc) / static_cast<double>(p.Q));
}

// Admitted debt of one pair (sparse_wrapper.py:3852-3859 -> 1755-1769).
__device__ __forceinline__ float admitted(float d, float dsum, float pc) {
  const float scale = pc / floor_tiny(dsum);
  return dsum > 0.f ? clamp01(d * scale) : 0.f;
}

// Global service gate (sparse_wrapper.py:3837-3842) from the per-head
// partials, summed in head order; every caller recomputes the same bits.
// One wave: lane h loads head h's partials (64 heads at a time), and the
// in-order float64 sums run over them lane by lane.
__device__ __forceinline__ int service_gate(const SelectParams &p, int lane) {
  if (!p.pending) return 0;
  double u = 0.0, w = 0.0, c = 0.0;
  for (int64_t h0 = 0; h0 < p.BH; h0 += 64) {
    const int64_t h = h0 + lane < p.BH ? h0 + lane : p.BH - 1;
    const double a = p.gate_part[3 * h + 0], b = p.gate_part[3 * h + 1], e = p.gate_part[3 * h + 2];
    const int n = p.BH - h0 < 64 ? static_cast<int>(p.BH - h0) : 64;
    for (int k = 0; k < n; ++k) {
      u = u + read_lane(a, k);
      w = w + read_lane(b, k);
      c = c + read_lane(e, k);
    }
  }
  const float fu = static_cast<float>(u), fw = static_cast<float>(w), fc = static_cast<float>(c);
  return (fc > 0.f) && (fu >= fw);
}

// ------------------------------------------------------------------ rows
// Row buffers: one per wave. The row starts at element off <= 3 and the
// 16-byte reads of a pass end at most 3 elements past off + K.
__host__ __device__ inline int64_t row_buf_elems(int64_t K) { return ((K + 6 + 3) / 4) * 4; }

// DMA of row [srow, srow + K) into buf: element k lands at buf[off + k] with
// off = (srow & 15) / 4, so every 16-byte chunk stays aligned. Whole chunks
// go by 16-byte DMA; the last 1-3 floats (when the row end is not 16-byte
// aligned) by 4-byte DMA, so nothing outside [srow & ~15, srow + K) is read.
// The caller waits with s_waitcnt vmcnt(0).
__device__ __forceinline__ int dma_row(const float *srow, int K, uint32_t *buf, int lane) {
  // srow and buf are uniform over the wave; make that explicit (the DMA
  // takes both in scalar registers).
  const uint64_t sr = reinterpret_cast<uint64_t>(srow);
  // (readfirstlane returns int: widen through uint32_t, never sign-extend)
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(sr >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(sr)));
  const uintptr_t start = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  const uintptr_t a0 = start & ~uintptr_t(15);
  const int off = static_cast<int>((start - a0) >> 2);
  const int bytes = static_cast<int>(start + static_cast<uintptr_t>(K) * 4u - a0);
  const int nchunks = bytes >> 4;
  const char *base = reinterpret_cast<const char *>(a0);
  const uint32_t lbase = __builtin_amdgcn_readfirstlane(lds_addr32(buf));
  for (int c0 = 0; c0 < nchunks; c0 += 64)
    if (c0 + lane < nchunks) lds_dma16(base, static_cast<uint32_t>(c0 + lane) * 16u, lbase + c0 * 16);
  const int tail = (bytes - (nchunks << 4)) >> 2;  // 0..3 floats
  if (lane < tail) lds_dma4(base + (nchunks << 4), lane * 4u, lbase + (nchunks << 4));
  return off;
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------------ arrival
// One workgroup per (32-row chunk, head). Wave w takes rows w, w+4, ... of
// the chunk: risk total (wave sum), conservative arrival A, pair arrival
// a_p = (A_2p + A_2p+1) / pair_size written in place over the row (position
// p was already consumed), its row sum (wave sum over the even positions).
// Then thread t adds the pair values of the four rows, in row order, into
// the float64 column partials of pairs t, t+256, ...
__global__ __launch_bounds__(1024) void arrival_kernel(const SelectParams p, int bufn) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  __shared__ int offs[16];
  const int nw = blockDim.x >> 6;  // waves per workgroup (4, 8 or 16)
  const int64_t chunk = blockIdx.x, bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform
  const int64_t q0 = chunk * kChunk;
  const int nrows = static_cast<int>(p.Q - q0 < kChunk ? p.Q - q0 : kChunk);
  const int K = static_cast<int>(p.K);
  const float *iota = p.innovation + bh * p.P;
  uint32_t *buf = lds + w * bufn;
  double part[kMaxPairsPerThread];
#pragma unroll
  for (int i = 0; i < kMaxPairsPerThread; ++i) part[i] = 0.0;

  for (int r0 = 0; r0 < nrows; r0 += nw) {
    const int r = r0 + w;
    if (r < nrows) {
      const int64_t row = bh * p.Q + q0 + r;
      const float *srow = p.score + row * p.K;
      const int off = dma_row(srow, K, buf, lane);
      wait_dma();
      const float *x = reinterpret_cast<const float *>(buf + off);
      int cap;
      if (p.row_cap) {
        cap = p.row_cap[row];
      } else {
        cap = p.topk < 1 ? 1 : p.topk;
        cap = cap > K ? K : cap;
        if (p.force_last && cap < K) {
          const uint32_t last = order_key(x[K - 1]);
          int beat = 0;
          for (int k = lane; k < K; k += 64) {
            const uint32_t kk = order_key(x[k]);
            beat += (kk > last) || (kk == last && k < K - 1);
          }
          cap += wave_sum_int(beat) >= cap ? 1 : 0;
        }
      }
      double acc = 0.0;
      for (int k = lane; k < K; k += 64) acc = acc + static_cast<double>(clean_score(x[k]) * iota[k >> 1]);
      const float total = static_cast<float>(wave_butterfly(acc));
      const float scale = static_cast<float>(cap) / floor_tiny(total);
      double racc = 0.0;
      float *apair = reinterpret_cast<float *>(buf + off);
      for (int kb = 0; kb < K; kb += 64) {
        const int k = kb + lane;
        float A = 0.f;
        if (k < K && total > 0.f) A = clamp01((clean_score(x[k]) * iota[k >> 1]) * scale);
        const float An = __shfl_down(A, 1);
        if (k < K && (lane & 1) == 0) {
          const float ap = (k + 1 < K) ? (A + An) / 2.0f : (A + 0.0f) / 1.0f;
          apair[k >> 1] = ap;
          racc = racc + static_cast<double>(ap);
        }
      }
      const float rowpair = static_cast<float>(wave_butterfly(racc));
      if (lane == 0) {
        p.total[row] = total;
        p.rowpair[row] = rowpair;
        p.cap[row] = cap;
        offs[w] = off;
      }
    }
    __syncthreads();
    const int rows_here = nrows - r0 < nw ? nrows - r0 : nw;
#pragma unroll
    for (int i = 0; i < kMaxPairsPerThread; ++i) {
      const int64_t pp = tid + static_cast<int64_t>(blockDim.x) * i;
      if (pp < p.P)
        for (int rr = 0; rr < rows_here; ++rr)
          part[i] = part[i] + static_cast<double>(__uint_as_float(lds[rr * bufn + offs[rr] + pp]));
    }
    __syncthreads();
  }
  double *out = p.part + (bh * p.nchunks + chunk) * p.P;
#pragma unroll
  for (int i = 0; i < kMaxPairsPerThread; ++i) {
    const int64_t pp = tid + static_cast<int64_t>(blockDim.x) * i;
    if (pp < p.P) out[pp] = part[i];
  }
}

// ------------------------------------------------------------------ head
// Per head, between the arrival and select passes: ledger settlement, pair
// capacity, admitted debt and the select pass's (innovation, admitted debt)
// table, the head's partials of the global gate; and the pending arrival
// (the mean over rows of the pair arrival). Workgroup 0 of a head settles all
// of its pairs (P <= 4096: eight per thread, every load in flight at once),
// keeps the settled debt, reflection and consumed service in LDS for wave 0's
// canonical wave sums, while wave 7 sums the pair capacity; the other
// workgroups take 512 pairs each for the pending arrival (the chunk partials,
// 64 loaded at a time, summed in chunk order).
constexpr int kHeadThreads = 512;
__global__ __launch_bounds__(kHeadThreads) void head_kernel(const SelectParams p) {
  extern __shared__ float hl[];  // workgroup 0: settled debt, reflection, consumed service (3 P floats)
  __shared__ float sh_pc, sh_dsum;
  const int64_t bh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t P = p.P;
  if (blockIdx.x > 0) {
    const int64_t pp = static_cast<int64_t>(blockIdx.x - 1) * kHeadThreads + tid;
    if (pp >= P) return;
    const double *part = p.part + bh * p.nchunks * P + pp;
    double acc = 0.0;
    for (int64_t c0 = 0; c0 < p.nchunks; c0 += 64) {
      double v[64];
#pragma unroll
      for (int u = 0; u < 64; ++u) v[u] = part[(c0 + u < p.nchunks ? c0 + u : p.nchunks - 1) * P];
#pragma unroll
      for (int u = 0; u < 64; ++u)
        if (c0 + u < p.nchunks) acc = acc + v[u];
    }
    p.arrival_out[bh * P + pp] = static_cast<float>(acc / static_cast<double>(p.Q));
    return;
  }
  float pc = 0.f;
  if (w == 7) pc = pair_capacity(p, bh, lane);
  float d[kSettleBatch], refl[kSettleBatch], sig[kSettleBatch], inn[kSettleBatch];
#pragma unroll
  for (int u = 0; u < kSettleBatch; ++u) {
    const int64_t j = tid + kHeadThreads * u < P ? tid + kHeadThreads * u : P - 1;
    inn[u] = p.innovation[bh * P + j];
  }
  settle_batch<kHeadThreads>(p, bh, tid, d, refl, sig);
#pragma unroll
  for (int u = 0; u < kSettleBatch; ++u) {
    const int64_t j = tid + kHeadThreads * u;
    if (j < P) {
      hl[j] = d[u];
      hl[P + j] = refl[u];
      hl[2 * P + j] = sig[u];
      p.debt_out[bh * P + j] = d[u];
      p.counts[bh * P + j] = 0;
    }
  }
  if (w == 7 && lane == 0) sh_pc = pc;
  __syncthreads();
  if (w == 0) {
    double dacc = 0.0, useful = 0.0, wasted = 0.0, consumed = 0.0;
    for (int64_t j = lane; j < P; j += 64) {
      const float dj = hl[j], rj = hl[P + j], sj = hl[2 * P + j];
      dacc = dacc + static_cast<double>(dj);
      useful = useful + static_cast<double>(clamp_min0(sj - rj));
      wasted = wasted + static_cast<double>(rj);
      consumed = consumed + static_cast<double>(sj);
    }
    const double ds = wave_butterfly(dacc);
    useful = wave_butterfly(useful);
    wasted = wave_butterfly(wasted);
    consumed = wave_butterfly(consumed);
    if (lane == 0) {
      sh_dsum = static_cast<float>(ds);
      p.gate_part[3 * bh + 0] = useful;
      p.gate_part[3 * bh + 1] = wasted;
      p.gate_part[3 * bh + 2] = consumed;
    }
  }
  __syncthreads();
  const float dsum = sh_dsum, pcap = sh_pc;
#pragma unroll
  for (int u = 0; u < kSettleBatch; ++u) {
    const int64_t j = tid + kHeadThreads * u;
    if (j < P) {
      const float admit = admitted(d[u], dsum, pcap);
      p.adm[bh * P + j] = admit;
      p.ia[bh * P + j] = float2{inn[u], admit};
    }
  }
}

// ------------------------------------------------------------------ select
// One wave per row with the row's keys in registers: lane l holds elements
// k = 256 i + 4 l + j (i < EPT / 4, j < 4), so each 16-byte load of a step
// is coalesced; key 0 (which no real value maps to) past the row end. Per
// row:
//   keys     order-preserving keys of the score (Top-K) or of the priority
//            (VASC) and the row's key range;
//   bracket  a 256-bin histogram of every 8th key over that range gives
//            lo <= hm1 with, very likely, fewer than c keys above hm1 and at
//            least c keys >= lo (sample ranks c S / K -+ 3 sigma + 1);
//   rank     histogram levels over the keys in [lo, hm1] (the whole range
//            when the bracket misses) find the c-th largest key exactly;
//   compact  the kept indices in ascending order, ties at the threshold
//            going to the lower index.
typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(4)));
typedef float floatx4u __attribute__((ext_vector_type(4), aligned(8)));

// Wave-uniform min and max of the keys in [lo, hi).
template <int EPT>
__device__ __forceinline__ void keys_minmax(const uint32_t (&key)[EPT], uint32_t lo, uint64_t hi, uint32_t &kmin,
                                            uint32_t &kmax) {
  uint32_t mn = 0xffffffffu, mx = 0u;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const bool in = key[j] >= lo && static_cast<uint64_t>(key[j]) < hi;
    mn = in && key[j] < mn ? key[j] : mn;
    mx = in && key[j] > mx ? key[j] : mx;
    if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t a = __shfl_xor(mn, o), b = __shfl_xor(mx, o);
    mn = a < mn ? a : mn;
    mx = b > mx ? b : mx;
  }
  kmin = __builtin_amdgcn_readfirstlane(mn);
  kmax = __builtin_amdgcn_readfirstlane(mx);
}

// 256-bin histogram (this wave's `hist`) of the keys in [kmin, kmin + 256 <<
// sh), read back as four bins per lane plus the inclusive suffix sum over
// lanes (keys in bins >= 4 lane).
__device__ __forceinline__ int hist_suffix(const uint32_t *hist, int lane, u32x4 &h) {
  h = *reinterpret_cast<const u32x4 *>(hist + 4 * lane);
  int suf = static_cast<int>(h[0] + h[1] + h[2] + h[3]);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_down(suf, o);
    if (lane + o < 64) suf += t;
  }
  return suf;
}

// Bin holding the r-th largest histogram entry (1 <= r <= total), or -1.
__device__ __forceinline__ int rank_bin(const u32x4 &h, int suf, int lane, int r) {
  int found = -1, above = suf;  // above: entries in bins >= the current one
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int next = above - static_cast<int>(h[b]);
    if (above >= r && next < r) found = 4 * lane + b;
    above = next;
  }
  const uint64_t bal = __builtin_amdgcn_ballot_w64(found >= 0);
  return bal ? __builtin_amdgcn_readlane(found, __builtin_ctzll(bal)) : -1;
}

// The r-th largest (1 <= r <= n) of n <= 64 keys, one per lane (lanes >= n
// hold none), all inside [lo, lo + 2^bits): the largest t with at least r keys
// >= t, built bit by bit from the top with ballot counts. Returns T and the
// numbers of keys above it (gt) and equal to it (eq).
__device__ __forceinline__ uint32_t rank_small(uint32_t mine, int n, int lane, uint32_t lo, int bits, int r, int &gt,
                                               int &eq) {
  const bool valid = lane < n;
  const uint32_t v = valid ? mine - lo : 0u;
  const uint64_t vm = __builtin_amdgcn_ballot_w64(valid);
  uint32_t pre = 0;
  for (int b = bits - 1; b >= 0; --b) {
    const uint32_t t = pre | (1u << b);
    if (__popcll(__builtin_amdgcn_ballot_w64(v >= t) & vm) >= r) pre = t;
  }
  gt = __popcll(__builtin_amdgcn_ballot_w64(v > pre) & vm);
  eq = __popcll(__builtin_amdgcn_ballot_w64(v == pre) & vm);
  return lo + pre;
}

// The c-th largest key (c >= 1) counting from the top of [kmin, kmax];
// keys above kmax are counted first. Each level histograms the keys of the
// current range into 256 bins of width 2^sh and takes the bin holding the
// rank; the search ends when that bin is kept whole, when its keys are all
// equal, or when it holds at most 64 keys (ranked exactly with readlane
// compares); otherwise the bin's own [min, max] is the next range. Returns
// false (nothing written) when the c-th largest key is not inside the
// first range. T: the threshold; need: how many keys equal to T to keep in
// index order (INT_MAX: all); eqT: how many keys equal T.
template <int EPT>
__device__ bool rank_keys(const uint32_t (&key)[EPT], int lane, uint32_t kmin, uint32_t kmax, int c, uint32_t *hist,
                          uint32_t *sbuf, uint32_t &T, int &need, int &eqT) {
  int above = 0;
#pragma unroll 1
  for (int level = 0;; ++level) {
    const uint32_t range = kmax - kmin;
    const int sh = 32 - __clz(range) > 8 ? 32 - __clz(range) - 8 : 0;
    *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{0, 0, 0, 0};
    wave_sync();
    int over = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      // branch-free: keys outside the range count into the lane's trash bin
      const uint32_t x = key[j];
      const bool in = x >= kmin && x <= kmax;
      atomicAdd(&hist[in ? (x - kmin) >> sh : 256u + lane], 1u);
      over += x > kmax;
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // keeps few element masks live
    }
    wave_sync();
    u32x4 h;
    const int suf = hist_suffix(hist, lane, h);
    const int inr = __builtin_amdgcn_readfirstlane(suf);
    if (level == 0) {
      above = __builtin_amdgcn_readfirstlane(wave_sum_int(over));
      if (c - above < 1 || c - above > inr) return false;
    }
    if (range == 0) {  // every key of the range is equal
      T = kmin;
      need = c - above;
      eqT = inr;
      return true;
    }
    const int need_r = c - above;
    const int bin = rank_bin(h, suf, lane, need_r);
    // keys in bins above `bin` and in `bin` itself
    int abv = 0, inb = 0;
    {
      int a = suf;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (4 * lane + b == bin) {
          inb = static_cast<int>(h[b]);
          abv = a - inb;
        }
        a -= static_cast<int>(h[b]);
      }
      const uint64_t bal = __builtin_amdgcn_ballot_w64(bin >= 4 * lane && bin < 4 * lane + 4);
      const int L = __builtin_ctzll(bal);
      abv = __builtin_amdgcn_readlane(abv, L);
      inb = __builtin_amdgcn_readlane(inb, L);
    }
    above += abv;
    const int need_b = c - above;  // 1 <= need_b <= inb
    const uint32_t lowT = kmin + (static_cast<uint32_t>(bin) << sh);
    const uint64_t highT = bin == 255 ? static_cast<uint64_t>(kmax) + 1u
                                      : static_cast<uint64_t>(kmin) + (static_cast<uint64_t>(bin + 1) << sh);
    if (need_b == inb) {
      T = lowT;
      need = 0x7fffffff;
      eqT = 0;
      return true;
    }
    if (inb <= 64) {
      // the bin's keys, one per lane (order irrelevant), then exact ranks
      int n = 0;
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        // branch-free: lanes without a bin key write their trash slot
        const bool in = key[j] >= lowT && static_cast<uint64_t>(key[j]) < highT;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
        sbuf[in ? n + lanes_below(bal) : 64 + lane] = key[j];
        n += __popcll(bal);
        if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
      wave_sync();
      int gt, eq;
      T = rank_small(lane < inb ? sbuf[lane] : 0u, inb, lane, lowT, sh, need_b, gt, eq);
      need = need_b - gt;
      eqT = eq;
      return true;
    }
    keys_minmax(key, lowT, highT, kmin, kmax);  // next level: the bin's own range
  }
}

// The c-th largest key (c >= 1) of the candidate keys in LDS, all inside
// [kmin, kmax]: lane l holds cnt of them at seg[0 .. cnt) (its own segment,
// maxcnt the wave's largest cnt). The histogram levels of rank_keys over
// the candidates; same outputs as rank_keys.
__device__ void rank_segs(const uint32_t *seg, int cnt, int maxcnt, int lane, uint32_t kmin, uint32_t kmax, int c,
                          uint32_t *hist, uint32_t *sbuf, uint32_t &T, int &need, int &eqT, int stride = 1) {
  int above = 0;
#pragma unroll 1
  for (;;) {
    const uint32_t range = kmax - kmin;
    const int sh = 32 - __clz(range) > 8 ? 32 - __clz(range) - 8 : 0;
    *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{0, 0, 0, 0};
    wave_sync();
    for (int r = 0; r < maxcnt; ++r) {
      const uint32_t x = r < cnt ? seg[r * stride] : 0u;
      const bool in = r < cnt && x >= kmin && x <= kmax;
      atomicAdd(&hist[in ? (x - kmin) >> sh : 256u + lane], 1u);
    }
    wave_sync();
    u32x4 h;
    const int suf = hist_suffix(hist, lane, h);
    const int inr = __builtin_amdgcn_readfirstlane(suf);
    if (range == 0) {
      T = kmin;
      need = c - above;
      eqT = inr;
      return;
    }
    const int need_r = c - above;
    const int bin = rank_bin(h, suf, lane, need_r);
    int abv = 0, inb = 0;
    {
      int a = suf;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        if (4 * lane + b == bin) {
          inb = static_cast<int>(h[b]);
          abv = a - inb;
        }
        a -= static_cast<int>(h[b]);
      }
      const int L = __builtin_ctzll(__builtin_amdgcn_ballot_w64(bin >= 4 * lane && bin < 4 * lane + 4));
      abv = __builtin_amdgcn_readlane(abv, L);
      inb = __builtin_amdgcn_readlane(inb, L);
    }
    above += abv;
    const int need_b = c - above;  // 1 <= need_b <= inb
    const uint32_t lowT = kmin + (static_cast<uint32_t>(bin) << sh);
    const uint64_t highT = bin == 255 ? static_cast<uint64_t>(kmax) + 1u
                                      : static_cast<uint64_t>(kmin) + (static_cast<uint64_t>(bin + 1) << sh);
    if (need_b == inb) {
      T = lowT;
      need = 0x7fffffff;
      eqT = 0;
      return;
    }
    if (inb <= 64) {
      int m = 0;
      for (int r = 0; r < maxcnt; ++r) {
        const uint32_t x = r < cnt ? seg[r * stride] : 0u;
        const bool in = r < cnt && x >= lowT && static_cast<uint64_t>(x) < highT;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
        sbuf[in ? m + lanes_below(bal) : 64 + lane] = x;
        m += __popcll(bal);
      }
      wave_sync();
      int gt, eq;
      T = rank_small(lane < inb ? sbuf[lane] : 0u, inb, lane, lowT, sh, need_b, gt, eq);
      need = need_b - gt;
      eqT = eq;
      return;
    }
    // next level: the bin's own key range
    uint32_t mn = 0xffffffffu, mx = 0u;
    for (int r = 0; r < maxcnt; ++r) {
      const uint32_t x = r < cnt ? seg[r * stride] : 0u;
      const bool in = r < cnt && x >= lowT && static_cast<uint64_t>(x) < highT;
      mn = in && x < mn ? x : mn;
      mx = in && x > mx ? x : mx;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t a = __shfl_xor(mn, o), b = __shfl_xor(mx, o);
      mn = a < mn ? a : mn;
      mx = b > mx ? b : mx;
    }
    kmin = __builtin_amdgcn_readfirstlane(mn);
    kmax = __builtin_amdgcn_readfirstlane(mx);
  }
}

// Sample-rank margin: 3 standard deviations of the count of S samples above
// a fraction f of the row, plus one.
__device__ __forceinline__ int sample_margin(int S, int c, int K) {
  const float f = static_cast<float>(c) / static_cast<float>(K);
  return static_cast<int>(3.f * __builtin_sqrtf(static_cast<float>(S) * f * (1.f - f))) + 1;
}

// Ascending compaction of the kept keys: element (lane, j) of a 256-element
// step follows every element of lower lanes and its own j' < j; ties at T
// are kept in index order up to need when split. The kept indices go to
// stage[0 ..) in LDS (other lanes write their trash slot stage[64 EPT +
// lane]). kMask: writes the 0/1 mask (every element of the row) instead.
// Returns the number kept.
template <bool kMask, int EPT>
__device__ __forceinline__ int compact_row(const uint32_t (&key)[EPT], int lane, uint32_t T, int need, bool split,
                                           bool none, uint32_t tsel, uint32_t *stage, uint8_t *mrow) {
  int run_sel = 0, run_eq = 0;
#pragma unroll
  for (int i = 0; i < EPT / 4; ++i) {
    bool sel[4];
    if (split) {
      bool eq[4];
      uint64_t beq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        eq[j] = key[4 * i + j] == T;
        beq[j] = __builtin_amdgcn_ballot_w64(eq[j]);
      }
      int eq_rank = run_eq;
#pragma unroll
      for (int j = 0; j < 4; ++j) eq_rank += lanes_below(beq[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sel[j] = key[4 * i + j] > T || (eq[j] && eq_rank < need);
        eq_rank += eq[j] ? 1 : 0;
        run_eq += __popcll(beq[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) sel[j] = !none && key[4 * i + j] >= tsel;
    }
    const int kk = 256 * i + 4 * lane;
    if (kMask) {
      // key 0 marks slots past the row end
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (key[4 * i + j] != 0u) mrow[kk + j] = sel[j] ? 1 : 0;
    } else {
      uint64_t bsel[4];
      int pos = run_sel;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bsel[j] = __builtin_amdgcn_ballot_w64(sel[j]);
        pos += lanes_below(bsel[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        stage[sel[j] ? pos : 64 * EPT + lane] = static_cast<uint32_t>(kk + j);
        pos += sel[j] ? 1 : 0;
        run_sel += __popcll(bsel[j]);
      }
    }
  }
  return run_sel;
}

// 256-element steps that are whole in every row an instance is launched for:
// launch_select_mode picks the instance for K in (64 * E', 64 * EPT], E'
// the next smaller instance, so the first E' / 4 steps never reach the row
// end and need no per-step branch.
template <int EPT>
constexpr int full_steps() {
  return EPT == 8 ? 1 : EPT == 12 ? 2 : EPT == 16 ? 3 : EPT == 24 ? 4 : EPT == 32 ? 6 : EPT == 36 ? 8
       : EPT == 48 ? 9 : EPT == 64 ? 12 : EPT == 96 ? 16 : EPT == 128 ? 24 : 0;
}

// per wave: histogram (256 bins + 64 per-lane trash bins), small-bin keys
// (64 + 64 per-lane trash slots), then 64 * (EPT + 1) words shared by the
// bracket candidates (one segment of EPT + 1 per lane) and the staged index
// list (K entries + 64 per-lane trash slots)
template <int EPT>
constexpr int wave_lds_words() {
  return 256 + 64 + 128 + 64 * (EPT + 1);
}

// kWaves waves per workgroup, rows_per_wave consecutive rows per wave (all
// rows of one head); LDS: the waves' histograms and small-bin buffers, then
// the workgroup's pair counts (VASC).
template <bool kVasc, int EPT>
__global__ __launch_bounds__(256) void select_kernel(const SelectParams p, int rows_per_wave) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint32_t *hist = lds + w * wave_lds_words<EPT>();
  uint32_t *sbuf = hist + 256 + 64;
  uint32_t *cand = sbuf + 128;
  uint32_t *pair_cnt = lds + kWaves * wave_lds_words<EPT>();
  const int64_t bh = blockIdx.y;
  const int K = static_cast<int>(p.K);
  int gate = 0;
  if (kVasc) {
    for (int64_t i = tid; i < (p.P + 1) / 2; i += 256) pair_cnt[i] = 0;  // packed pair counts
    __syncthreads();
    gate = service_gate(p, lane0);
  }
  const float2 *ia = kVasc ? p.ia + bh * p.P : nullptr;
  const uint32_t top = order_key(kFltMax);
  // the forced value (protected / forced last blocks) is left out of the
  // bracket histogram's range, which it would otherwise stretch
  const uint32_t forced = kVasc ? top : 0xffffffffu;

  for (int rr = 0; rr < rows_per_wave; ++rr) {
    const int64_t q = (static_cast<int64_t>(blockIdx.x) * kWaves + w) * rows_per_wave + rr;
    if (q >= p.Q) break;
    const int64_t row = bh * p.Q + q;
    const float *srow = p.score + row * p.K;
    // An opaque copy of the lane index: per-element indices and masks are
    // recomputed in every row instead of being hoisted out of the row loop
    // (64-bit masks for every element would spill).
    int lane = lane0;
    asm volatile("" : "+v"(lane));

    // ---- load and keys. Whether a 256-element step lies wholly inside the
    // row is wave-uniform, so the branches are scalar and every load of the
    // row is issued before the first wait; in the step holding the row end
    // each element loads from a clamped (in-bounds) index.
    uint32_t key[EPT];
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      const int kk = 256 * i + 4 * lane;
      if (i < full_steps<EPT>() || 256 * (i + 1) <= K) {
        const u32x4u x = *reinterpret_cast<const u32x4u *>(srow + kk);
#pragma unroll
        for (int j = 0; j < 4; ++j) key[4 * i + j] = x[j];
      } else if (256 * i < K) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = kk + j;
          const uint32_t v = __float_as_uint(srow[k < K ? k : K - 1]);
          key[4 * i + j] = k < K ? v : 0u;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) key[4 * i + j] = 0u;
      }
    }
    int c;
    float total = 0.f, scale = 0.f;
    uint32_t last = 0;
    if (kVasc) {
      const int cap = p.cap[row];
      c = cap < p.max_capacity ? cap : p.max_capacity;
      total = p.total[row];
      scale = static_cast<float>(cap) / floor_tiny(total);
    } else {
      // per-row counts (cdf threshold) or the uniform budget; the index
      // width was sized for max_capacity (plus the forced tail)
      c = p.row_cap ? p.row_cap[row] : p.topk;
      c = c < 1 ? 1 : c;
      const int lim = p.max_capacity >= K ? K : p.max_capacity - p.force_last;
      if (p.row_cap) c = c < lim ? c : lim;
      c = c > K ? K : c;
      last = order_key(srow[K - 1]);
    }
    uint32_t kmin = 0xffffffffu, kmax = 0u, kmaxh = 0u;
    uint32_t rawmax = 0u;  // Top-K: largest raw score bits (sign set or NaN above 0x7f800000)
    int beat = 0;
    // Steps wholly before the last element need no per-element masks; only
    // the step holding the last element (K - 1) checks k < K and k == K - 1
    // (which step that is, is wave-uniform).
    auto transform = [&](const int i, auto edge_c) {
      constexpr bool kEdge = decltype(edge_c)::value;
      const int kk = 256 * i + 4 * lane;
      // (innovation, admitted debt) of the step's two pairs kk/2, kk/2 + 1
      // (pair indices clamped into [0, P) in the step holding the row end)
      floatx4 pa = {0.f, 0.f, 0.f, 0.f};
      if (kVasc) {
        if (!kEdge) {
          const floatx4u x = *reinterpret_cast<const floatx4u *>(ia + (kk >> 1));
          pa = floatx4{x[0], x[1], x[2], x[3]};
        } else {
          const int P = (K + 1) >> 1, p0 = kk >> 1;
          const float2 x0 = ia[p0 < P ? p0 : P - 1], x1 = ia[p0 + 1 < P ? p0 + 1 : P - 1];
          pa = floatx4{x0.x, x0.y, x1.x, x1.y};
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = kk + j;
        const bool ok = !kEdge || k < K;
        const bool is_last = kEdge && k == K - 1;
        const float sv = __uint_as_float(key[4 * i + j]);
        uint32_t kj;
        if (kVasc) {
          const float pin = pa[2 * (j >> 1)], pad = pa[2 * (j >> 1) + 1];
          const float A = total > 0.f ? clamp01((clean_score(sv) * pin) * scale) : 0.f;
          kj = order_key(gate ? A + pad : A);
          if (p.protected_mask) kj = ok && p.protected_mask[row * p.K + k] ? top : kj;
          kj = p.force_last && is_last ? top : kj;
          // execution priority (non-negative, or FLT_MAX when protected):
          // the key with the sign bit cleared is its float bits
          if (p.priority_out && ok) p.priority_out[row * p.K + k] = __uint_as_float(kj & 0x7fffffffu);
        } else {
          // the raw bits with the sign flipped: the order key of any
          // non-negative, non-NaN score (others are redone below)
          const uint32_t raw = key[4 * i + j];
          rawmax = ok && raw > rawmax ? raw : rawmax;
          kj = raw ^ 0x80000000u;
          if (p.force_last) {
            beat += ok && ((kj > last) || (kj == last && !is_last)) ? 1 : 0;
            kj = is_last ? 0xffffffffu : kj;
          }
        }
        kj = ok ? kj : 0u;
        kmin = ok && kj < kmin ? kj : kmin;
        kmax = kj > kmax ? kj : kmax;
        kmaxh = kj != forced && kj > kmaxh ? kj : kmaxh;
        key[4 * i + j] = kj;
      }
    };
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      if (i < full_steps<EPT>() || 256 * (i + 1) < K)
        transform(i, std::false_type{});
      else if (256 * i < K)
        transform(i, std::true_type{});
    }
    if (!kVasc) {
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t a = __shfl_xor(rawmax, o);
        rawmax = a > rawmax ? a : rawmax;
      }
      if (__builtin_amdgcn_readfirstlane(rawmax) > 0x7f800000u) {
        // a negative, -0 or NaN score: full order keys for the row
        kmin = 0xffffffffu;
        kmax = kmaxh = 0u;
        beat = 0;
#pragma unroll
        for (int i = 0; i < EPT / 4; ++i) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int k = 256 * i + 4 * lane + j;
            const bool ok = k < K;
            uint32_t kj = order_key(__uint_as_float(key[4 * i + j] ^ 0x80000000u));
            if (p.force_last) {
              beat += ok && ((kj > last) || (kj == last && k != K - 1)) ? 1 : 0;
              kj = k == K - 1 ? 0xffffffffu : kj;
            }
            kj = ok ? kj : 0u;
            kmin = ok && kj < kmin ? kj : kmin;
            kmax = kj > kmax ? kj : kmax;
            kmaxh = kj != forced && kj > kmaxh ? kj : kmaxh;
            key[4 * i + j] = kj;
          }
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const uint32_t a = __shfl_xor(kmin, o), b = __shfl_xor(kmax, o), d = __shfl_xor(kmaxh, o);
      kmin = a < kmin ? a : kmin;
      kmax = b > kmax ? b : kmax;
      kmaxh = d > kmaxh ? d : kmaxh;
    }
    kmin = __builtin_amdgcn_readfirstlane(kmin);
    kmax = __builtin_amdgcn_readfirstlane(kmax);
    kmaxh = __builtin_amdgcn_readfirstlane(kmaxh);
    if (kmaxh < kmin) kmaxh = kmax;  // every key is forced
    if (!kVasc && p.force_last && c < K) c += wave_sum_int(beat) >= c ? 1 : 0;
    c = c < 0 ? 0 : (c > K ? K : c);
    c = __builtin_amdgcn_readfirstlane(c);  // wave-uniform: keeps the control flow below scalar
    const bool all = c >= K, none = c == 0;

    // ---- threshold: keys > T kept, keys == T kept in index order up to need
    uint32_t T = 1u;
    int need = 0x7fffffff, eqT = 0;
    if (none) T = 0xffffffffu;
    if (!all && !none) {
      // bracket from every 8th key (steps i even, j == 0)
      const uint32_t range = kmaxh - kmin;
      const int sh = 32 - __clz(range) > 8 ? 32 - __clz(range) - 8 : 0;
      *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{0, 0, 0, 0};
      wave_sync();
#pragma unroll
      for (int i = 0; i < EPT / 4; i += 2) {
        const uint32_t x = key[4 * i];
        atomicAdd(&hist[x != 0u && x <= kmaxh ? (x - kmin) >> sh : 256u + lane], 1u);
      }
      wave_sync();
      u32x4 h;
      const int suf = hist_suffix(hist, lane, h);
      const int S = __builtin_amdgcn_readfirstlane(suf);
      const int rs = static_cast<int>(static_cast<int64_t>(c) * S / K);
      const int m = sample_margin(S, c, K);
      const int bin_hi = rs - m >= 1 ? rank_bin(h, suf, lane, rs - m) : -1;
      const int bin_lo = rs + m <= S ? rank_bin(h, suf, lane, rs + m) : -1;
      uint32_t hm1 = kmax, lo = kmin;  // keys > hm1 kept outright; candidates in [lo, hm1]
      if (bin_hi >= 0 && bin_hi < 255) {
        const uint64_t e = static_cast<uint64_t>(kmin) + (static_cast<uint64_t>(bin_hi + 1) << sh);
        if (e <= kmaxh) hm1 = static_cast<uint32_t>(e - 1);
      }
      if (bin_lo >= 0) lo = kmin + (static_cast<uint32_t>(bin_lo) << sh);
      if (lo > hm1) lo = kmin;
      // candidates [lo, hm1] to LDS, each lane into its own segment (every
      // key is written at the segment's end, which only advances past a
      // candidate), keys above hm1 counted
      uint32_t *seg = cand + lane * (EPT + 1);
      int above = 0, cnt = 0;
      const uint32_t span = hm1 - lo;
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const uint32_t x = key[j];
        above += x > hm1;
        seg[cnt] = x;
        cnt += x - lo <= span;  // key 0 (and anything below lo) wraps above span
      }
      above = __builtin_amdgcn_readfirstlane(wave_sum_int(above));
      int n = cnt, maxcnt = cnt;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        n += __shfl_xor(n, o);
        maxcnt = max(maxcnt, __shfl_xor(maxcnt, o));
      }
      n = __builtin_amdgcn_readfirstlane(n);
      maxcnt = __builtin_amdgcn_readfirstlane(maxcnt);
      wave_sync();
      if (above < c && above + n >= c)
        rank_segs(seg, cnt, maxcnt, lane, lo, hm1, c - above, hist, sbuf, T, need, eqT);
      else  // missed bracket: rank the whole row
        rank_keys(key, lane, kmin, kmax, c, hist, sbuf, T, need, eqT);
    }
    const bool split = !all && !none && need < eqT;
    const uint32_t tsel = all ? 1u : T;  // keys >= tsel are kept (no split)

    // ---- ascending compaction (indices and pair counts), then the optional
    // mask and priority outputs in passes of their own
    int32_t *irow = p.index_out + row * p.width;
    asm volatile("" : "+v"(lane));  // element indices recomputed here, not kept from the loads
    const int run_sel = compact_row<false, EPT>(key, lane, T, need, split, none, tsel, cand, nullptr);
    wave_sync();
    // the staged list to the index row (coalesced) and, for VASC, into the
    // workgroup's pair counts: two 16-bit counts per word (pair p in half
    // p % 2 of word p / 2; a workgroup's rows give each pair at most
    // 2 * rows_per_workgroup)
    for (int e = lane; e < run_sel; e += 64) {
      const uint32_t kb = cand[e];
      if (e < p.width) irow[e] = static_cast<int32_t>(kb);
      if (kVasc) atomicAdd(&pair_cnt[kb >> 2], 1u << ((kb & 2u) << 3));
    }
    wave_sync();  // the staged list is read before the next row reuses it
    if (p.mask_out)
      compact_row<true, EPT>(key, lane, T, need, split, none, tsel, nullptr, p.mask_out + row * p.K);
    for (int i = lane; i < p.sink && run_sel + i < p.width; i += 64) irow[run_sel + i] = static_cast<int32_t>(p.K + i);
    for (int64_t e = run_sel + p.sink + lane; e < p.width; e += 64) irow[e] = -1;  // the rest of the row defined
    if (lane == 0) p.count_out[row] = run_sel + p.sink;
  }
  if (kVasc) {
    __syncthreads();
    for (int64_t i = tid; i < p.P; i += 256) {
      const uint32_t v = (pair_cnt[i >> 1] >> ((i & 1) << 4)) & 0xffffu;
      if (v) atomicAdd(&p.counts[bh * p.P + i], static_cast<int32_t>(v));
    }
  }
}

// ------------------------------------------------------------------ service
__global__ __launch_bounds__(256) void service_kernel(const SelectParams p) {
  // the gate flag: wave 0 of workgroup 0 (the gate's sums take a whole wave)
  if (p.gate_out && blockIdx.x == 0 && threadIdx.x < 64) {
    const int g = service_gate(p, static_cast<int>(threadIdx.x));
    if (threadIdx.x == 0) *p.gate_out = g;
  }
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= p.BH * p.P) return;
  const int64_t pp = i % p.P;
  const float pair_size = (p.K % 2 && pp == p.P - 1) ? 1.0f : 2.0f;
  const float denom = pair_size * static_cast<float>(p.Q);
  p.service_out[i] = static_cast<float>(p.counts[i]) / denom;
}

// ============================================================ register rows
// Kernels for rows of at most 4096 key blocks with the row in registers in
// the lane order of the canonical wave sum: lane j holds element k = j + 64 m
// in slot m < EPT. The row is padded to 64 EPT elements: loads past its end
// read +0.0 through the buffer range check, so a padding element has score
// and risk +0 and contributes +0.0 to every sum (which leaves a float64 sum
// of non-negative terms bit-identical). In the selection a padding element
// has the smallest key of its row (priority +0, or key 0 on the general
// paths) and a larger index than every real element, so with ties going to
// the lower index it is never among the top c <= K: the per-element code
// needs no bounds masks.
//
// Fast path: a row whose scores are finite and non-negative (raw bits below
// 0x7f800000: no NaN, infinity, negative value or -0.0), in a head whose
// innovations are finite, with a finite risk total and a finite scale. Its
// risks, conservative arrivals and priorities are then finite and
// non-negative, so clean_score is the identity, clamp01 is a minimum with 1
// and the order key of a priority is its bits with the sign bit set; the
// arithmetic and its roundings are the general path's.
constexpr uint32_t kFinite = 0x7f800000u;  // raw bits of +inf

// The lane index through an empty asm: per-element indices and masks made
// from it are recomputed in the loop that uses them instead of being hoisted
// out of the row loop and held (64-bit masks for every slot would spill).
__device__ __forceinline__ int opaque_lane(int lane) {
  asm volatile("" : "+v"(lane));
  return lane;
}

// x[m] = src[lane + 64 m] for lane + 64 m < n, +0.0 past n, through buffer
// resources rebased every 16 slots (every offset is 4 lane plus an immediate).
template <int EPT>
__device__ __forceinline__ void load_slots(float (&x)[EPT], const float *src, int n, int lane) {
#pragma unroll
  for (int g = 0; g < (EPT + 15) / 16; ++g) {
    const int left = n - 1024 * g;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(src + (left > 0 ? 1024 * g : 0)), 0, left > 0 ? 4 * left : 0, 0x00020000);
#pragma unroll
    for (int m = 16 * g; m < EPT && m < 16 * g + 16; ++m)
      x[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 4 * lane + 256 * (m - 16 * g), 0, 0));
  }
}

// Arrival: one workgroup per (32-row chunk, head), kRowWaves row waves; each
// wave takes rows w, w + kRowWaves, ... of the chunk. Per row: capacity, risk
// total, conservative arrival, pair arrivals (to the wave's LDS row, 32 EPT
// wide so the padding's pairs land in its tail) and their row sum; then the
// chunk's float64 column partials in row order, as arrival_kernel. Also
// records per row whether the select pass may take the fast path (flags).
template <int EPT, int kRowWaves>
__global__ __launch_bounds__(64 * kRowWaves) __attribute__((amdgpu_waves_per_eu(EPT <= 33 ? 4 : 2)))
void arrival_rows_kernel(const SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) float alds[];
  constexpr int kThreads = 64 * kRowWaves;
  constexpr int kStride = 32 * EPT;  // LDS row of pair arrivals
  constexpr int kPairs = (kStride + kThreads - 1) / kThreads;  // column partials per thread
  const int P = static_cast<int>(p.P), K = static_cast<int>(p.K);
  // chunks run from the last down, every head's chunk c together: the select
  // pass sweeps each head's rows upward, so each pass starts on the rows the
  // other read last, which the Infinity Cache may still hold
  const int64_t lin = blockIdx.x, bh = lin % p.BH, chunk = p.nchunks - 1 - lin / p.BH;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t q0 = chunk * kChunk;
  const int nrows = static_cast<int>(p.Q - q0 < kChunk ? p.Q - q0 : kChunk);
  const bool even = (lane & 1) == 0;
  // the head's innovations (0 past the pairs), read per element as pin[(lane >> 1) + 32 m],
  // and whether all are finite
  float *pin = alds + kRowWaves * kStride;
  bool bad = false;
  for (int i = tid; i < kStride; i += kThreads) {
    const float v = i < P ? p.innovation[bh * P + i] : 0.f;
    pin[i] = v;
    bad |= !(v <= kFltMax);
  }
  const bool head_fast = !__syncthreads_or(bad);
  double part[kPairs];
#pragma unroll
  for (int i = 0; i < kPairs; ++i) part[i] = 0.0;
  float *ap_row = alds + w * kStride;
  const float *pin_l = pin + (lane >> 1);

  float x[EPT];
  for (int r0 = 0; r0 < nrows; r0 += kRowWaves) {
    if (r0 + w < nrows) {
      const int64_t row = bh * p.Q + q0 + r0 + w;
      const float *srow = p.score + row * p.K;
      load_slots(x, srow, K, lane);
      int cap;
      if (p.row_cap) {
        cap = p.row_cap[row];
      } else {
        cap = p.topk < 1 ? 1 : p.topk;
        cap = cap > K ? K : cap;
        if (p.force_last && cap < K) {
          const uint32_t last = order_key(srow[K - 1]);
          const int ln = opaque_lane(lane);
          int beat = 0;
#pragma unroll
          for (int m = 0; m < EPT; ++m) {
            const int k = ln + 64 * m;
            const uint32_t kk = order_key(x[m]);
            beat += k < K && ((kk > last) || (kk == last && k < K - 1));
          }
          cap += wave_sum_int(beat) >= cap ? 1 : 0;
        }
      }
      uint32_t hi = 0u;
#pragma unroll
      for (int m = 0; m < EPT; ++m) hi = max(hi, __float_as_uint(x[m]));
      const bool clean = head_fast && __builtin_amdgcn_ballot_w64(hi >= kFinite) == 0;
      // risks (in place) and their canonical sum
      double acc = 0.0;
      // (the innovation reads are fenced in groups of four slots, so that few
      // of them hold registers at a time)
      if (clean) {
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          x[m] = x[m] * pin_l[32 * m];
          acc = acc + static_cast<double>(x[m]);
          if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          x[m] = clean_score(x[m]) * pin_l[32 * m];
          acc = acc + static_cast<double>(x[m]);
          if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      }
      const double tot = wave_butterfly(acc);
      const float total = static_cast<float>(tot);
      const float scale = static_cast<float>(cap) / floor_tiny(total);
      const bool live = total > 0.f;
      // every risk finite (a sum of finite non-negative floats stays far below the float64 limit)
      const bool fast = clean && tot <= 1.0e300 && scale <= kFltMax;
      double racc = 0.0;
      if (fast && !(K & 1)) {
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          const float A = live ? fminf(x[m] * scale, 1.0f) : 0.f;
          const float ap = (A + dpp<kQuadXor1>(A)) * 0.5f;  // both lanes of a pair form its sum (addition commutes)
          racc = racc + static_cast<double>(even ? ap : 0.f);
          x[m] = ap;
        }
      } else {
        const int ln = opaque_lane(lane);
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          const int k = ln + 64 * m;
          const float A = live && k < K ? (fast ? fminf(x[m] * scale, 1.0f) : clamp01(x[m] * scale)) : 0.f;
          const float s2 = A + dpp<kQuadXor1>(A);
          const float ap = k == K - 1 ? s2 : s2 * 0.5f;  // an odd tail pairs with itself: (A + 0) / 1
          racc = racc + static_cast<double>(even ? ap : 0.f);
          x[m] = ap;
        }
      }
      if (even) {
#pragma unroll
        for (int m = 0; m < EPT; ++m) ap_row[(lane >> 1) + 32 * m] = x[m];
      }
      const float rowpair = static_cast<float>(wave_butterfly(racc));
      if (lane == 0) {
        p.total[row] = total;
        p.rowpair[row] = rowpair;
        p.cap[row] = cap;
        p.flags[row] = fast ? 1 : 0;
      }
    }
    __syncthreads();
    const int rows_here = nrows - r0 < kRowWaves ? nrows - r0 : kRowWaves;
    int t = tid;
    asm volatile("" : "+v"(t));  // addresses made here, not held across the row loop
#pragma unroll
    for (int i = 0; i < kPairs; ++i) {
      const int pp = t + kThreads * i;
      if (pp < P)
        for (int rr = 0; rr < rows_here; ++rr) part[i] = part[i] + static_cast<double>(alds[rr * kStride + pp]);
    }
    __syncthreads();
  }
  double *out = p.part + (bh * p.nchunks + chunk) * p.P;
#pragma unroll
  for (int i = 0; i < kPairs; ++i) {
    const int pp = tid + kThreads * i;
    if (pp < P) out[pp] = part[i];
  }
}

// Candidate keys staged by the select pass: one list per wave, filled slot
// by slot in lane order; up to kListCap of them (more: the row is ranked on
// its registers instead), with room for one more slot's 64 past the cap.
constexpr int kSeg = 16;
constexpr int kListCap = 64 * kSeg - 64;
// per wave: histogram (256 bins + 64 per-lane trash bins), 64 gathered keys
// (+ 64 trash slots), the candidate list (64 kSeg words)
constexpr int kRowWaveWords = 320 + 128 + 64 * kSeg;

// The threshold of the keys of a padded row (64 EPT keys, 0 the smallest
// any element can have, held by the padding): keys > T are kept, keys == T
// in index order up to need (eqT of them). A histogram of a sample (every
// lane's slots 0, 4, 8, ...; 256 bins over the sampled keys' range above 0)
// brackets the c-th largest key at its sample rank c S / n -+ 3 sigma + 1
// (a quarter of the keys sampled: about 2 n 3 sqrt(f (1 - f) / S)
// candidates, about 330 at 4096 keys and f = c / n = 1/4, well under
// kListCap); keys above the bracket are kept, the bracket's keys go to the
// wave's candidate list and are ranked exactly (rank_segs). When fewer than
// c keys exceed 0 the threshold is 0, its ties going in index order. When
// the bracket misses, or holds more than kListCap keys, the threshold is
// found by bisection over the key bits.
constexpr int kSampleStep = 4;  // sampled slots: m = 0, 4, 8, ...
template <int EPT>
__device__ __forceinline__ void rows_threshold(const uint32_t (&key)[EPT], int lane, int c, uint32_t *hist,
                                               uint32_t *sbuf, uint32_t *cand, uint32_t &T, int &need, int &eqT) {
  constexpr int n = 64 * EPT;
  constexpr int S = 64 * ((EPT + kSampleStep - 1) / kSampleStep);  // samples
  uint32_t smin = 0xffffffffu, smax = 0u;  // smin: over sampled keys above 0, less one
#pragma unroll
  for (int m = 0; m < EPT; m += kSampleStep) {
    smin = min(smin, key[m] - 1u);
    smax = max(smax, key[m]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    smin = min(smin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(smin), o)));
    smax = max(smax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(smax), o)));
  }
  smin = __builtin_amdgcn_readfirstlane(smin) + 1u;  // 0 when no sampled key exceeds 0
  smax = __builtin_amdgcn_readfirstlane(smax);
  uint32_t hm1 = 0xffffffffu, lo = 1u;  // keys > hm1 kept outright; candidates in [lo, hm1]
  const int rs = static_cast<int>(static_cast<int64_t>(c) * S / n);
  const int mg = sample_margin(S, c, n);
  if (smin != 0u && smax > smin) {
    const uint32_t range = smax - smin;
    const int sh = 32 - __clz(range) > 8 ? 32 - __clz(range) - 8 : 0;
    *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{0, 0, 0, 0};
    wave_sync();
#pragma unroll
    for (int m = 0; m < EPT; m += kSampleStep) atomicAdd(&hist[key[m] ? (key[m] - smin) >> sh : 256u + lane], 1u);
    wave_sync();
    u32x4 h;
    const int suf = hist_suffix(hist, lane, h);
    const int spos = __builtin_amdgcn_readfirstlane(suf);  // sampled keys above 0
    if (rs - mg >= 1 && rs - mg <= spos) {
      const int b = rank_bin(h, suf, lane, rs - mg);
      if (b < 255) hm1 = smin + ((static_cast<uint32_t>(b) + 1u) << sh) - 1u;
    }
    if (rs + mg <= spos) lo = smin + (static_cast<uint32_t>(rank_bin(h, suf, lane, rs + mg)) << sh);
    if (lo > hm1) lo = 1u;
  }
  // candidates [lo, hm1] appended to the wave's list slot by slot (each
  // lane at its rank among the slot's candidate lanes; nothing is written
  // once kListCap is passed); keys above hm1 counted
  const uint32_t span = hm1 - lo;
  int above = 0, tot = 0;  // wave-uniform
  uint32_t *trash = sbuf + 64 + lane;
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    const uint32_t x = key[m];
    above += __popcll(__builtin_amdgcn_ballot_w64(x > hm1));
    const bool in = x - lo <= span;  // keys below lo (0 among them) wrap above span
    const uint64_t b = __builtin_amdgcn_ballot_w64(in);
    // branch-free: every lane writes, the non-candidates to their trash slot;
    // past kListCap the slot's candidates overwrite the list's last 64 entries
    const uint32_t pos = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b), 0u));
    uint32_t *at = (cand + (tot < kListCap ? tot : kListCap)) + pos;
    *(in ? at : trash) = x;
    tot += __popcll(b);
  }
  wave_sync();
  if (above < c && above + tot >= c && tot <= kListCap) {
    // lane l ranks list entries l, l + 64, ...
    const int cnt = lane < tot ? (tot - lane + 63) / 64 : 0;
    rank_segs(cand + lane, cnt, (tot + 63) / 64, lane, lo, hm1, c - above, hist, sbuf, T, need, eqT, 64);
    return;
  }
  if (above + tot < c && lo == 1u) {  // every key above 0 is kept; the rest of the c are 0 keys
    T = 0u;
    need = c - above - tot;
    eqT = n - above - tot;
    return;
  }
  // the bracket missed, or held more than kListCap keys: the c-th largest
  // key by bisection over its bits (the largest t with at least c keys >= t),
  // exact for any distribution and holding no more registers than the keys
  uint32_t pre = 0u;
  for (int b = 31; b >= 0; --b) {
    const uint32_t t = pre | (1u << b);
    int ge = 0;
#pragma unroll
    for (int m = 0; m < EPT; ++m) ge += __popcll(__builtin_amdgcn_ballot_w64(key[m] >= t));
    if (ge >= c) pre = t;
  }
  int gt = 0, eq = 0;
#pragma unroll
  for (int m = 0; m < EPT; ++m) {
    gt += __popcll(__builtin_amdgcn_ballot_w64(key[m] > pre));
    eq += __popcll(__builtin_amdgcn_ballot_w64(key[m] == pre));
  }
  T = pre;
  need = c - gt;
  eqT = eq;
}

// Select: one wave per row, rows_per_wave consecutive rows per wave, the
// workgroup's rows in one head. Keys in registers in the arrival's lane
// order (kPrefetch: the next row's scores load while this row is ranked);
// on the fast paths a key is the raw bits of the non-negative priority or
// score, otherwise its order key (the padding's key is 0 either way). VASC:
// the (innovation, admitted debt) table of the head and the pair counts live
// in LDS. Index lists are written in ascending order straight from the
// ballots: the selected lanes of a slot store at their rank among them past
// the slot's base (in the store's scalar offset) and count their pair.
template <bool kVasc, int EPT, bool kPrefetch>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(EPT <= 33 ? 4 : 1)))
void select_rows_kernel(const SelectParams p, int rows_per_wave, int row_step) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = static_cast<int>(p.K), P = static_cast<int>(p.P);
  uint32_t *hist = lds + w * kRowWaveWords;
  uint32_t *sbuf = hist + 320;
  uint32_t *cand = sbuf + 128;
  uint32_t *pair_cnt = lds + kWaves * kRowWaveWords;  // 32 EPT words, one per pair (VASC)
  float2 *ia_s = reinterpret_cast<float2 *>(pair_cnt + 32 * EPT);  // 32 EPT entries (VASC), 0 past P
  const int64_t bh = blockIdx.y;
  // this wave's rows: q_first + rr row_step, rr < rows_per_wave (consecutive
  // rows when row_step is 1, else every row_step-th row of the head)
  const int64_t wave_id = static_cast<int64_t>(blockIdx.x) * kWaves + w;
  const int64_t q_first = row_step == 1 ? wave_id * rows_per_wave : wave_id;
  // the first row's scores load while the head's tables are set up (rows of
  // up to 33 elements per lane: wider rows would lose a wave per SIMD to the
  // registers held across the set-up)
  constexpr bool kEarly = kPrefetch || EPT <= 33;
  float x[EPT], nxt[EPT];
  if (kEarly && q_first < p.Q) load_slots(kPrefetch ? nxt : x, p.score + (bh * p.Q + q_first) * p.K, K, lane0);
  int gate = 0;
  bool ia_fast = true;
  if (kVasc) {
    // the head's table entries of this thread (indices clamped into the
    // head; entries past P are zero), loaded before the gate's sums so that
    // all the loads are in flight together
    constexpr int kT = (32 * EPT + 255) / 256;
    float2 t_ia[kT];
#pragma unroll
    for (int t = 0; t < kT; ++t) t_ia[t] = p.ia[bh * P + (tid + 256 * t < P ? tid + 256 * t : P - 1)];
    gate = service_gate(p, lane0);
    bool bad = false;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      const int i = tid + 256 * t;
      if (i < 32 * EPT) {
        const float2 v = i < P ? t_ia[t] : float2{0.f, 0.f};
        ia_s[i] = v;
        bad |= !(v.y <= kFltMax);
        pair_cnt[i] = 0u;
      }
    }
    ia_fast = !__syncthreads_or(bad);
  }

  for (int rr = 0; rr < rows_per_wave; ++rr) {
    const int64_t q = q_first + static_cast<int64_t>(rr) * row_step;
    if (q >= p.Q) break;
    // lane-derived values and masks are recomputed per row, not held across rows
    const int lane = opaque_lane(lane0);
    const int64_t row = bh * p.Q + q;
    const float *srow = p.score + row * p.K;
    if (kPrefetch) {
#pragma unroll
      for (int m = 0; m < EPT; ++m) x[m] = nxt[m];
      if (rr + 1 < rows_per_wave && q + row_step < p.Q) load_slots(nxt, srow + row_step * p.K, K, lane);
    } else if (rr > 0 || !kEarly) {
      load_slots(x, srow, K, lane);
    }
    // ---- keys
    uint32_t key[EPT];
    int c;
    bool exact_keys;  // order keys, real elements masked against the row end
    if (kVasc) {
      const int cap = p.cap[row];
      c = cap < p.max_capacity ? cap : p.max_capacity;
      const float total = p.total[row];
      const float scale = static_cast<float>(cap) / floor_tiny(total);
      const bool live = total > 0.f;
      // with the gate on and K odd, the padding element K shares pair P - 1's admitted debt,
      // so its fast-path key would not be the row's smallest: the masked path handles it
      exact_keys = !(p.flags[row] && (gate == 0 || (ia_fast && (K & 1) == 0)));
      const float2 *ia_l = ia_s + (lane >> 1);
      // (the table reads are fenced in groups of four slots, so that few of
      // them hold registers at a time)
      if (!exact_keys) {
        if (!live) {
#pragma unroll
          for (int m = 0; m < EPT; ++m) {
            key[m] = gate ? __float_as_uint(ia_l[32 * m].y) : 0u;
            if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
          }
        } else if (gate) {
#pragma unroll
          for (int m = 0; m < EPT; ++m) {
            const float2 ia = ia_l[32 * m];
            key[m] = __float_as_uint(fminf((x[m] * ia.x) * scale, 1.0f) + ia.y);
            if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int m = 0; m < EPT; ++m) {
            key[m] = __float_as_uint(fminf((x[m] * ia_l[32 * m].x) * scale, 1.0f));
            if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
          }
        }
      } else {
        const int ln = opaque_lane(lane);
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          const int k = ln + 64 * m;
          const float2 ia = ia_l[32 * m];
          const float A = live ? clamp01((clean_score(x[m]) * ia.x) * scale) : 0.f;
          key[m] = k < K ? order_key(gate ? A + ia.y : A) : 0u;
          if ((m & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (p.priority_out) {
        const int ln = opaque_lane(lane);
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
          const int k = ln + 64 * m;
          if (k < K) p.priority_out[row * p.K + k] = __uint_as_float(exact_keys ? key[m] & 0x7fffffffu : key[m]);
        }
      }
    } else {
      c = p.row_cap ? p.row_cap[row] : p.topk;
      c = c < 1 ? 1 : c;
      const int lim = p.max_capacity >= K ? K : p.max_capacity;
      if (p.row_cap) c = c < lim ? c : lim;
      c = c > K ? K : c;
      uint32_t hi = 0u;
#pragma unroll
      for (int m = 0; m < EPT; ++m) hi = max(hi, __float_as_uint(x[m]));
      // non-negative, non-NaN scores (+inf included) order as their bits
      exact_keys = __builtin_amdgcn_ballot_w64(hi > kFinite) != 0;
      if (!exact_keys) {
#pragma unroll
        for (int m = 0; m < EPT; ++m) key[m] = __float_as_uint(x[m]);
      } else {
        const int ln = opaque_lane(lane);
#pragma unroll
        for (int m = 0; m < EPT; ++m) key[m] = ln + 64 * m < K ? order_key(x[m]) : 0u;
      }
    }
    c = c < 0 ? 0 : (c > K ? K : c);
    c = __builtin_amdgcn_readfirstlane(c);

    // ---- threshold: keys > T kept, keys == T kept in index order up to need
    uint32_t T = 0xffffffffu;  // c == 0: nothing is kept (no key reaches T with need 0)
    int need = 0, eqT = 1;
    if (c > 0) rows_threshold(key, lane, c, hist, sbuf, cand, T, need, eqT);
    const bool split = need < eqT;

    // ---- ascending compaction straight to the index row and pair counts
    const __amdgpu_buffer_rsrc_t irs =
        __builtin_amdgcn_make_buffer_rsrc(p.index_out + row * p.width, 0, static_cast<int>(4 * p.width), 0x00020000);
    uint32_t *cnt_l = pair_cnt + (lane >> 1);
    int base = 0;  // wave-uniform
    // one element slot: its ballot; the selected lanes store their index at
    // base + their rank among the slot's selected lanes (base in the store's
    // scalar offset) and count their pair
    auto emit = [&](int m, bool sel) {
      const uint64_t bm = __builtin_amdgcn_ballot_w64(sel);
      const uint32_t pos = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0u));
      // branch-free: the unselected lanes store past the buffer range, which drops them
      __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(lane + 64 * m), irs, sel ? 4 * pos : 0x7ffffff0u,
                                            4 * base, 0);
      if (kVasc) atomicAdd(&cnt_l[32 * m], sel ? 1u : 0u);
      base += __popcll(bm);
    };
    if (!split) {
#pragma unroll
      for (int m = 0; m < EPT; ++m) emit(m, key[m] >= T);
    } else {
      int run_eq = 0;
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const uint32_t xk = key[m];
        const bool eq = xk == T;
        const uint64_t beq = __builtin_amdgcn_ballot_w64(eq);
        int below = lanes_below(beq);
        asm volatile("" : "+v"(below));
        emit(m, xk > T || (eq && run_eq + below < need));
        run_eq += __popcll(beq);
      }
    }
    if (p.mask_out) {
      uint8_t *mrow = p.mask_out + row * p.K;
      const int ln = opaque_lane(lane);
      int run_eq = 0;
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const int k = ln + 64 * m;
        const uint32_t xk = key[m];
        bool sel = xk >= T;
        if (split) {
          const bool eq = xk == T;
          const uint64_t beq = __builtin_amdgcn_ballot_w64(eq);
          sel = xk > T || (eq && run_eq + lanes_below(beq) < need);
          run_eq += __popcll(beq);
        }
        if (k < K) mrow[k] = sel ? 1 : 0;
      }
    }
    int32_t *irow = p.index_out + row * p.width;
    for (int i = lane; i < p.sink && base + i < p.width; i += 64) irow[base + i] = static_cast<int32_t>(p.K + i);
    for (int64_t e = base + p.sink + lane; e < p.width; e += 64) irow[e] = -1;  // the rest of the row defined
    if (lane == 0) p.count_out[row] = base + p.sink;
  }
  if (kVasc) {
    __syncthreads();
    for (int64_t i = tid; i < p.P; i += 256)
      if (pair_cnt[i]) atomicAdd(&p.counts[bh * p.P + i], static_cast<int32_t>(pair_cnt[i]));
  }
}

// ------------------------------------------------------------------ order
// The selector's priority order: per row the M largest priorities, largest
// first, equal priorities in ascending block index (the selected indices,
// priority.topk(M, sorted=True).indices). One wave per row. The M blocks come
// from the select pass's index list when the row kept exactly M patch blocks
// (its kept set is the top M under the same tie rule); otherwise the row's
// order keys go to registers (k = lane + 64 m, padding 0), rows_threshold
// finds the M-th largest key and the M blocks go to LDS in ascending index
// order. Up to 1024 blocks are then sorted in registers (a bitonic network
// over 64-bit composites key << 32 | ~block, descending, so equal keys end in
// ascending block order); more take a stable LSD radix sort in LDS over the
// key bytes that differ among them (descending digits; stability keeps equal
// keys in ascending block order). Per wave, after the rank buffers: the
// (key, block) buffers of M rounded up to 64 entries (two for the radix sort).

// One stable pass over n (key, block) pairs from (sk, sv) to (dk, dv),
// descending in the key byte at `shift`. `hist`: 256 words of this wave.
__device__ void order_pass(const uint32_t *sk, const uint32_t *sv, uint32_t *dk, uint32_t *dv, int n, int shift,
                           uint32_t *hist, int lane) {
  *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{0, 0, 0, 0};
  wave_sync();
  for (int i = lane; i < n; i += 64) atomicAdd(&hist[255u - ((sk[i] >> shift) & 255u)], 1u);
  wave_sync();
  // exclusive prefix of the digit counts: four bins per lane, then across lanes
  const u32x4 h = *reinterpret_cast<const u32x4 *>(hist + 4 * lane);
  const int own = static_cast<int>(h[0] + h[1] + h[2] + h[3]);
  int inc = own;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  const uint32_t e = static_cast<uint32_t>(inc - own);
  *reinterpret_cast<u32x4 *>(hist + 4 * lane) = u32x4{e, e + h[0], e + h[0] + h[1], e + h[0] + h[1] + h[2]};
  wave_sync();
  const uint64_t lt = lanemask_lt();
  for (int b0 = 0; b0 < n; b0 += 64) {
    const int i = b0 + lane;
    const bool valid = i < n;
    const uint32_t kk = valid ? sk[i] : 0u, vv = valid ? sv[i] : 0u;
    const uint32_t d = 255u - ((kk >> shift) & 255u);
    // the valid lanes holding the same digit
    uint64_t same = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bb = __builtin_amdgcn_ballot_w64(bit);
      same &= bit ? bb : ~bb;
    }
    const uint32_t off = valid ? hist[d] : 0u;
    wave_sync();  // every lane has read its digit's offset before the highest lane advances it
    if (valid) {
      const uint32_t at = off + static_cast<uint32_t>(__popcll(same & lt));
      dk[at] = kk;
      dv[at] = vv;
      if ((same >> lane) == 1u) hist[d] = off + static_cast<uint32_t>(__popcll(same));
    }
    wave_sync();
  }
}

__device__ __forceinline__ uint64_t xor_lane64(uint64_t v, int off) {
  const uint64_t lo = xor_lane(static_cast<uint32_t>(v), off), hi = xor_lane(static_cast<uint32_t>(v >> 32), off);
  return (hi << 32) | lo;
}

// Descending bitonic sort of 64 NPL composites, element e = NPL lane + j.
// A merge step at STRIDE inside blocks of SIZE leaves the larger value at
// the lower element of each pair in descending blocks ((e & SIZE) == 0),
// the smaller in ascending ones. Levels and steps recurse at compile time.
template <int NPL, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_step(uint64_t (&v)[NPL], int lane) {
  if constexpr (STRIDE >= NPL) {
    constexpr int lo = STRIDE / NPL;
    const bool lower = (lane & lo) == 0;
    const bool desc = (lane & (SIZE / NPL)) == 0;  // SIZE >= 2 NPL here
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const uint64_t o = xor_lane64(v[j], lo);
      const bool big = v[j] > o;
      v[j] = (lower == desc) == big ? v[j] : o;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      if (j & STRIDE) continue;
      const bool desc = SIZE < NPL ? (j & SIZE) == 0 : (lane & (SIZE / NPL)) == 0;
      const uint64_t a = v[j], b = v[j ^ STRIDE];
      const bool swap = desc ? a < b : a > b;
      v[j] = swap ? b : a;
      v[j ^ STRIDE] = swap ? a : b;
    }
  }
  if constexpr (STRIDE > 1) bitonic_step<NPL, SIZE, STRIDE / 2>(v, lane);
}

template <int NPL, int SIZE = 2>
__device__ __forceinline__ void bitonic_desc(uint64_t (&v)[NPL], int lane) {
  bitonic_step<NPL, SIZE, SIZE / 2>(v, lane);
  if constexpr (SIZE < 64 * NPL) bitonic_desc<NPL, SIZE * 2>(v, lane);
}

__device__ __forceinline__ uint64_t order_composite(uint32_t key, uint32_t block) {
  return (static_cast<uint64_t>(key) << 32) | static_cast<uint64_t>(0xffffffffu - block);
}

// NPL: sorted entries per lane (64 NPL >= M), 0 for the radix sort in LDS.
// index / count / width / sink: the select pass's lists (index may be null).
template <int EPT, int NPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(EPT <= 33 ? 4 : 1)))
void order_rows_kernel(const float *prio, const int32_t *index, const int32_t *count, int64_t width, int sink,
                       int64_t rows, int K, int M, int wave_words, int64_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane0 = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + w;
  if (row >= rows) return;
  uint32_t *hist = lds + static_cast<int64_t>(w) * wave_words;
  uint32_t *sbuf = hist + 320;
  uint32_t *cand = sbuf + 128;
  const int Mp = (M + 63) & ~63;
  uint32_t *k0 = cand + 64 * kSeg, *v0 = k0 + Mp;
  const int lane = opaque_lane(lane0);
  const float *prow = prio + row * K;
  const int listed = index ? __builtin_amdgcn_readfirstlane(count[row] - sink) : -1;
  constexpr int kRegs = NPL > 0 ? NPL : 1;
  uint64_t v[kRegs];
  if (NPL > 0 && listed == M) {
    // the select pass's kept blocks (ascending; block ids clamped into the row)
    const int32_t *irow = index + row * width;
#pragma unroll
    for (int j = 0; j < kRegs; ++j) {
      const int e = NPL * lane + j;
      int blk = e < M ? irow[e] : 0;
      blk = blk < 0 ? 0 : (blk >= K ? K - 1 : blk);
      v[j] = e < M ? order_composite(order_key(prow[blk]), static_cast<uint32_t>(blk)) : 0u;
    }
  } else {
    if (listed == M) {
      const int32_t *irow = index + row * width;
      for (int i = lane; i < M; i += 64) {
        int blk = irow[i];
        blk = blk < 0 ? 0 : (blk >= K ? K - 1 : blk);
        k0[i] = order_key(prow[blk]);
        v0[i] = static_cast<uint32_t>(blk);
      }
    } else {
      float x[EPT];
      load_slots(x, prow, K, lane);
      uint32_t key[EPT];
#pragma unroll
      for (int m = 0; m < EPT; ++m) key[m] = lane + 64 * m < K ? order_key(x[m]) : 0u;
      // keys > T kept, keys == T in index order up to need (M >= 1: T is a real key)
      uint32_t T = 0xffffffffu;
      int need = 0, eqT = 1;
      rows_threshold(key, lane, M, hist, sbuf, cand, T, need, eqT);
      const bool split = need < eqT;
      int base = 0, run_eq = 0;
#pragma unroll
      for (int m = 0; m < EPT; ++m) {
        const uint32_t xk = key[m];
        bool sel = xk >= T;
        if (split) {
          const bool eq = xk == T;
          const uint64_t beq = __builtin_amdgcn_ballot_w64(eq);
          sel = xk > T || (eq && run_eq + lanes_below(beq) < need);
          run_eq += __popcll(beq);
        }
        const uint64_t bm = __builtin_amdgcn_ballot_w64(sel);
        if (sel) {
          const int at = base + lanes_below(bm);
          k0[at] = xk;
          v0[at] = static_cast<uint32_t>(lane + 64 * m);
        }
        base += __popcll(bm);
      }
    }
    wave_sync();
    if (NPL > 0) {
#pragma unroll
      for (int j = 0; j < kRegs; ++j) {
        const int e = NPL * lane + j;
        v[j] = e < M ? order_composite(k0[e], v0[e]) : 0u;
      }
    }
  }
  int64_t *orow = out + row * M;
  if (NPL > 0) {
    bitonic_desc<kRegs>(v, lane);
#pragma unroll
    for (int j = 0; j < kRegs; ++j) {
      const int e = NPL * lane + j;
      if (e < M) orow[e] = static_cast<int64_t>(0xffffffffu - static_cast<uint32_t>(v[j]));
    }
    return;
  }
  // radix: the kept keys lie in [min, max]; bytes above the highest bit where
  // those differ are common to all of them and need no pass
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  for (int i = lane; i < M; i += 64) {
    kmin = k0[i] < kmin ? k0[i] : kmin;
    kmax = k0[i] > kmax ? k0[i] : kmax;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t a = static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmin), o));
    const uint32_t b = static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmax), o));
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  const uint32_t diff = __builtin_amdgcn_readfirstlane(kmax ^ kmin);
  const int passes = diff ? (31 - __clz(static_cast<int>(diff))) / 8 + 1 : 0;
  uint32_t *sk = k0, *sv = v0, *dk = v0 + Mp, *dv = v0 + 2 * Mp;
  for (int ps = 0; ps < passes; ++ps) {
    order_pass(sk, sv, dk, dv, M, 8 * ps, hist, lane);
    uint32_t *t = sk;
    sk = dk;
    dk = t;
    t = sv;
    sv = dv;
    dv = t;
  }
  for (int i = lane; i < M; i += 64) orow[i] = static_cast<int64_t>(sv[i]);
}

__global__ void settle_terminal_kernel(const float *debt_in, const float *pending, const float *service, int64_t n,
                                       float *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float d = debt_in ? clamp_min0(debt_in[i]) : 0.f;
  out[i] = clamp_min0((d + pending[i]) - service[i]);
}

struct Workspace {
  size_t total, rowpair, cap, adm, ia, part, gate_part, counts, flags, bytes;
};

Workspace layout(int64_t B, int64_t H, int64_t Q, int64_t K) {
  const size_t BH = static_cast<size_t>(B * H), P = static_cast<size_t>((K + 1) / 2);
  Workspace w;
  size_t off = 0;
  w.total = off;     off += align256(BH * Q * 4);
  w.rowpair = off;   off += align256(BH * Q * 4);
  w.cap = off;       off += align256(BH * Q * 4);
  w.adm = off;       off += align256(BH * P * 4);
  w.ia = off;        off += align256(BH * P * 8);
  w.part = off;      off += align256(BH * static_cast<size_t>(cdiv(Q, kChunk)) * P * 8);
  w.gate_part = off; off += align256(BH * 3 * 8);
  w.counts = off;    off += align256(BH * P * 4);
  w.flags = off;     off += align256(BH * Q * 4);
  w.bytes = off;
  return w;
}

int reserve_lds(const void *kern, size_t lds_bytes) {
  if (lds_bytes <= 64 * 1024) return VASC_OK;
  const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_bytes));
  if (e != hipSuccess) {
    set_error("vasc_select_blocks: cannot reserve %zu bytes of LDS: %s", lds_bytes, hipGetErrorString(e));
    return VASC_ERR_HIP;
  }
  return VASC_OK;
}

template <bool kVasc, int EPT>
int launch_select_cfg(const SelectParams &p, hipStream_t s) {
  // Rows per wave: enough waves to give every SIMD several (1..4 rows);
  // VASC accumulates pair counts per workgroup, so more rows per workgroup
  // keep the global count atomics down.
  const int64_t rows = p.BH * p.Q;
  const int rpw = static_cast<int>(rows >= 4 * 8192 ? 4 : (rows >= 2 * 8192 ? 2 : 1));
  const size_t lds_bytes =
      (static_cast<size_t>(kWaves) * wave_lds_words<EPT>() + (kVasc ? static_cast<size_t>(p.P + 1) / 2 : 0)) * 4;
  const void *kern = reinterpret_cast<const void *>(select_kernel<kVasc, EPT>);
  int rc;
  if ((rc = reserve_lds(kern, lds_bytes))) return rc;
  const dim3 grid(static_cast<unsigned>(cdiv(p.Q, static_cast<int64_t>(kWaves) * rpw)), static_cast<unsigned>(p.BH));
  hipLaunchKernelGGL((select_kernel<kVasc, EPT>), grid, dim3(256), lds_bytes, s, p, rpw);
  return check_launch("vasc_select_blocks/select");
}

// Keys per lane: the row rounded up to whole 256-element steps.
template <bool kVasc>
int launch_select_mode(const SelectParams &p, hipStream_t s) {
  const int64_t K = p.K;
  if (K <= 256) return launch_select_cfg<kVasc, 4>(p, s);
  if (K <= 512) return launch_select_cfg<kVasc, 8>(p, s);
  if (K <= 768) return launch_select_cfg<kVasc, 12>(p, s);
  if (K <= 1024) return launch_select_cfg<kVasc, 16>(p, s);
  if (K <= 1536) return launch_select_cfg<kVasc, 24>(p, s);
  if (K <= 2048) return launch_select_cfg<kVasc, 32>(p, s);
  if (K <= 2304) return launch_select_cfg<kVasc, 36>(p, s);
  if (K <= 3072) return launch_select_cfg<kVasc, 48>(p, s);
  if (K <= 4096) return launch_select_cfg<kVasc, 64>(p, s);
  if (K <= 6144) return launch_select_cfg<kVasc, 96>(p, s);
  return launch_select_cfg<kVasc, 128>(p, s);
}

// Register-row select for K <= 4096 (not with protected blocks or a forced
// last block, which the staged kernel handles).
// Workgroups of a register-row select kernel resident on the device at once
// (queried once per kernel instantiation).
template <bool kVasc, int EPT, typename Kern>
int resident_workgroups(Kern kern, size_t lds_bytes) {
  static std::atomic<int> cached{0};
  int r = cached.load(std::memory_order_relaxed);
  if (r) return r;
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds_bytes) != hipSuccess)
    cus = per_cu = 0;
  r = cus * per_cu > 0 ? cus * per_cu : 1024;
  cached.store(r, std::memory_order_relaxed);
  return r;
}

// The rows of a head are dealt to its waves round-robin over a grid of at
// most one resident round of workgroups (its share of the device per head),
// so no partial second round of whole waves follows the first: a wave's
// rows differ in number by at most one.
template <bool kVasc, int EPT>
int launch_select_rows_cfg(const SelectParams &p, hipStream_t s) {
  constexpr bool kPrefetch = false;
  // per wave rank buffers; VASC: pair counts (32 EPT words) and the (innovation, debt) table (32 EPT float2)
  const size_t lds_bytes = static_cast<size_t>(kWaves) * kRowWaveWords * 4 + (kVasc ? 384 * static_cast<size_t>(EPT) : 0);
  auto kern = select_rows_kernel<kVasc, EPT, kPrefetch>;
  int rc;
  if ((rc = reserve_lds(reinterpret_cast<const void *>(kern), lds_bytes))) return rc;
  const int64_t per_head = cdiv(static_cast<int64_t>(resident_workgroups<kVasc, EPT>(kern, lds_bytes)), p.BH);
  const int64_t need = cdiv(p.Q, static_cast<int64_t>(kWaves));
  const int64_t gx = per_head < need ? per_head : need;
  const int step = static_cast<int>(gx * kWaves);
  const int rpw = static_cast<int>(cdiv(p.Q, static_cast<int64_t>(step)));
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(p.BH));
  hipLaunchKernelGGL(kern, grid, dim3(256), lds_bytes, s, p, rpw, step);
  return check_launch("vasc_select_blocks/select");
}

template <bool kVasc>
int launch_select_rows(const SelectParams &p, hipStream_t s) {
  const int64_t K = p.K;
  if (K <= 256) return launch_select_rows_cfg<kVasc, 4>(p, s);
  if (K <= 576) return launch_select_rows_cfg<kVasc, 9>(p, s);
  if (K <= 768) return launch_select_rows_cfg<kVasc, 12>(p, s);
  if (K <= 1088) return launch_select_rows_cfg<kVasc, 17>(p, s);
  if (K <= 1536) return launch_select_rows_cfg<kVasc, 24>(p, s);
  if (K <= 2112) return launch_select_rows_cfg<kVasc, 33>(p, s);
  if (K <= 3072) return launch_select_rows_cfg<kVasc, 48>(p, s);
  return launch_select_rows_cfg<kVasc, 64>(p, s);
}

// Priority order: as many row waves per workgroup (up to 4) as keep the
// workgroup's LDS within 64 KB; a single wave takes more (up to 137 KB at
// 8192 blocks).
struct OrderArgs {
  const float *prio;
  const int32_t *index, *count;
  int64_t width;
  int sink;
  int64_t rows;
  int K, M;
  int64_t *out;
};

template <int EPT, int NPL>
int launch_order_cfg(const OrderArgs &a, hipStream_t s) {
  const int wave_words = kRowWaveWords + (NPL > 0 ? 2 : 4) * ((a.M + 63) & ~63);
  const size_t wave_bytes = static_cast<size_t>(wave_words) * 4;
  int waves = static_cast<int>((64 * 1024) / wave_bytes);
  waves = waves < 1 ? 1 : (waves > kWaves ? kWaves : waves);
  const size_t lds_bytes = wave_bytes * waves;
  const void *kern = reinterpret_cast<const void *>(order_rows_kernel<EPT, NPL>);
  int rc;
  if ((rc = reserve_lds(kern, lds_bytes))) return rc;
  hipLaunchKernelGGL((order_rows_kernel<EPT, NPL>), dim3(static_cast<unsigned>(cdiv(a.rows, waves))),
                     dim3(64 * waves), lds_bytes, s, a.prio, a.index, a.count, a.width, a.sink, a.rows, a.K, a.M,
                     wave_words, a.out);
  return check_launch("vasc_priority_order");
}

// Sorted entries per lane: the fewest that hold M (rows of K <= 64 EPT keys
// hold M <= K); the radix sort past 1024.
template <int EPT>
int launch_order_npl(const OrderArgs &a, hipStream_t s) {
  if (a.M <= 64) return launch_order_cfg<EPT, 1>(a, s);
  if (a.M <= 128) return launch_order_cfg<EPT, 2>(a, s);
  if constexpr (64 * EPT <= 256) {
    return launch_order_cfg<EPT, 4>(a, s);
  } else {
    if (a.M <= 256) return launch_order_cfg<EPT, 4>(a, s);
    if (a.M <= 512) return launch_order_cfg<EPT, 8>(a, s);
    if constexpr (64 * EPT <= 1024) {
      return launch_order_cfg<EPT, 16>(a, s);
    } else {
      if (a.M <= 1024) return launch_order_cfg<EPT, 16>(a, s);
      return launch_order_cfg<EPT, 0>(a, s);
    }
  }
}

int launch_order(const OrderArgs &a, hipStream_t s) {
  if (a.K <= 256) return launch_order_npl<4>(a, s);
  if (a.K <= 576) return launch_order_npl<9>(a, s);
  if (a.K <= 1088) return launch_order_npl<17>(a, s);
  if (a.K <= 2112) return launch_order_npl<33>(a, s);
  if (a.K <= 4096) return launch_order_npl<64>(a, s);
  return launch_order_npl<128>(a, s);
}

// Register rows serve both modes up to 4096 key blocks; protected blocks, a
// forced last block and wider rows take the staged kernel.
int launch_select(const SelectParams &p, bool vasc, hipStream_t s) {
  if (!p.protected_mask && !p.force_last && p.K <= 64 * 64)
    return vasc ? launch_select_rows<true>(p, s) : launch_select_rows<false>(p, s);
  return vasc ? launch_select_mode<true>(p, s) : launch_select_mode<false>(p, s);
}

// Rows of up to 36 elements per lane fit in 128 VGPRs: eight row waves per
// chunk then give four waves per SIMD on grids of a few hundred chunks; rows
// of up to 16 elements (K <= 1024, grids of ~150 chunks at C2) take sixteen.
// Wider rows keep four row waves (two waves per SIMD, register bound).
template <int EPT>
int launch_arrival_rows_cfg(const SelectParams &p, hipStream_t s) {
  constexpr int kRowWaves = EPT <= 17 ? 16 : (EPT <= 33 ? 8 : 4);
  // pair arrivals per row wave, then the innovation table
  const size_t lds_bytes = static_cast<size_t>(kRowWaves + 1) * 32 * EPT * 4;
  const void *kern = reinterpret_cast<const void *>(arrival_rows_kernel<EPT, kRowWaves>);
  int rc;
  if ((rc = reserve_lds(kern, lds_bytes))) return rc;
  hipLaunchKernelGGL((arrival_rows_kernel<EPT, kRowWaves>),
                     dim3(static_cast<unsigned>(p.nchunks * p.BH)), dim3(64 * kRowWaves), lds_bytes,
                     s, p);
  return VASC_OK;
}
int launch_arrival_rows(const SelectParams &p, hipStream_t s) {
  const int64_t K = p.K;
  if (K <= 256) return launch_arrival_rows_cfg<4>(p, s);
  if (K <= 576) return launch_arrival_rows_cfg<9>(p, s);
  if (K <= 1088) return launch_arrival_rows_cfg<17>(p, s);
  if (K <= 1536) return launch_arrival_rows_cfg<24>(p, s);
  if (K <= 2112) return launch_arrival_rows_cfg<33>(p, s);
  if (K <= 3072) return launch_arrival_rows_cfg<48>(p, s);
  return launch_arrival_rows_cfg<64>(p, s);
}

int launch_rows(const SelectParams &p, bool vasc, hipStream_t s) {
  const int64_t bufn = row_buf_elems(p.K);
  int rc;
  if (vasc) {
    if (p.K <= 64 * 64) {
      if ((rc = launch_arrival_rows(p, s))) return rc;
    } else {
      // As many waves per chunk (16, 8 or 4) as keep the row buffers within
      // 64 KB; the column partials then need P <= 16 * (64 * waves).
      int aw = 16;
      while (aw > 4 && static_cast<size_t>(aw) * bufn * 4 > 64 * 1024) aw >>= 1;
      const size_t lds_bytes = static_cast<size_t>(aw) * bufn * 4;
      if ((rc = reserve_lds(reinterpret_cast<const void *>(arrival_kernel), lds_bytes))) return rc;
      hipLaunchKernelGGL(arrival_kernel, dim3(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.BH)),
                         dim3(64 * aw), lds_bytes, s, p, static_cast<int>(bufn));
    }
    if ((rc = check_launch("vasc_select_blocks/arrival"))) return rc;
    // workgroup 0 of a head settles its ledger, the others take 512 pairs each of the pending arrival
    hipLaunchKernelGGL(head_kernel, dim3(static_cast<unsigned>(1 + cdiv(p.P, kHeadThreads)), static_cast<unsigned>(p.BH)),
                       dim3(kHeadThreads), static_cast<size_t>(3 * p.P) * sizeof(float), s, p);
    if ((rc = check_launch("vasc_select_blocks/head"))) return rc;
  }
  if ((rc = launch_select(p, vasc, s))) return rc;
  if (vasc) {
    hipLaunchKernelGGL(service_kernel, dim3(static_cast<unsigned>(cdiv(p.BH * p.P, 256))), dim3(256), 0, s, p);
    if ((rc = check_launch("vasc_select_blocks/service"))) return rc;
  }
  return VASC_OK;
}

}  // namespace
}  // namespace vasc

extern "C" size_t vasc_select_workspace_size(int64_t B, int64_t H, int64_t q_blocks, int64_t k_blocks) {
  if (B <= 0 || H <= 0 || q_blocks <= 0 || k_blocks <= 0) return 0;
  return vasc::layout(B, H, q_blocks, k_blocks).bytes;
}

extern "C" int64_t vasc_select_workspace_offset(int64_t B, int64_t H, int64_t q_blocks, int64_t k_blocks,
                                                int32_t region) {
  if (B <= 0 || H <= 0 || q_blocks <= 0 || k_blocks <= 0) return -1;
  const vasc::Workspace w = vasc::layout(B, H, q_blocks, k_blocks);
  switch (region) {
    case VASC_WS_ROW_TOTAL: return static_cast<int64_t>(w.total);
    case VASC_WS_ROW_PAIR_SUM: return static_cast<int64_t>(w.rowpair);
    case VASC_WS_ROW_CAPACITY: return static_cast<int64_t>(w.cap);
    case VASC_WS_ADMITTED_DEBT: return static_cast<int64_t>(w.adm);
    default: return -1;
  }
}

namespace vasc {
namespace {

// Byte ranges [a, a + n) and [b, b + n) overlap (NULL never overlaps).
bool overlaps(const void *a, const void *b, size_t n) {
  if (!a || !b) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + n && y < x + n;
}

int select_blocks_impl(const float *score, const float *innovation, int64_t B, int64_t H, int64_t Q, int64_t K,
                       int32_t mode, int32_t topk, const int32_t *row_cap, const uint8_t *protected_mask,
                       int32_t force_last, int32_t max_capacity, int32_t sink_blocks, const float *debt_in,
                       const float *pending_arrival, const float *prev_service, float *debt_out,
                       float *arrival_out, float *service_out, int32_t *gate_out, float *priority_out,
                       uint8_t *mask_out, int32_t *index_out, int64_t width, int32_t *count_out, void *workspace,
                       size_t workspace_bytes, void *stream) {
  VASC_REQUIRE(score && index_out && count_out, "score, index_out and count_out are required");
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(score) & 15) == 0, "score must be 16-byte aligned");
  VASC_REQUIRE(B > 0 && H > 0 && Q > 0 && K > 0, "sizes must be positive");
  VASC_SUPPORTED(K <= 8192, "K=%lld key blocks not built (built: <= 8192)", (long long)K);
  VASC_REQUIRE(mode == VASC_MODE_TOPK || mode == VASC_MODE_VASC, "unknown mode %d", mode);
  VASC_REQUIRE(sink_blocks >= 0, "sink_blocks must be non-negative");
  VASC_REQUIRE(B * H < 65536, "B*H too large");
  VASC_REQUIRE(Q < (int64_t(1) << 31) / kWaves, "Q too large");
  const bool vasc = mode == VASC_MODE_VASC;
  int64_t maxc;
  if (vasc) {
    VASC_REQUIRE(innovation && debt_out && arrival_out && service_out, "VASC needs innovation and state outputs");
    VASC_REQUIRE(max_capacity >= 0, "max_capacity must be non-negative");
    VASC_REQUIRE(!prev_service || pending_arrival, "prev_service without pending_arrival");
    // The head pass reads every ledger input of a head while other
    // workgroups write that head's outputs: in-place updates would race.
    const size_t ledger = static_cast<size_t>(B * H * ((K + 1) / 2)) * sizeof(float);
    const float *ins[3] = {debt_in, pending_arrival, prev_service};
    const float *outs[3] = {debt_out, arrival_out, service_out};
    for (const float *o : outs)
      for (const float *i : ins)
        VASC_REQUIRE(!overlaps(o, i, ledger), "ledger outputs must not overlap the ledger inputs");
    VASC_REQUIRE(!overlaps(debt_out, arrival_out, ledger) && !overlaps(debt_out, service_out, ledger) &&
                     !overlaps(arrival_out, service_out, ledger),
                 "ledger outputs must not overlap each other");
    maxc = max_capacity < K ? max_capacity : K;
  } else {
    // row_cap: per-row counts, each at most max_capacity (K when 0)
    int64_t t = row_cap ? (max_capacity > 0 ? max_capacity : K) : (topk < 1 ? 1 : topk);
    maxc = t + (force_last ? 1 : 0);
    maxc = maxc < K ? maxc : K;
  }
  VASC_REQUIRE(width >= maxc + sink_blocks, "index width %lld < max count %lld", (long long)width,
               (long long)(maxc + sink_blocks));
  SelectParams p;
  p.score = score;
  p.innovation = innovation;
  p.BH = B * H;
  p.Q = Q;
  p.K = K;
  p.P = (K + 1) / 2;
  p.mode = mode;
  p.topk = topk;
  p.force_last = force_last;
  p.max_capacity = static_cast<int32_t>(maxc);
  p.sink = sink_blocks;
  p.row_cap = row_cap;
  p.protected_mask = protected_mask;
  p.debt_in = debt_in;
  p.pending = pending_arrival;
  p.prev_service = prev_service;
  p.debt_out = debt_out;
  p.arrival_out = arrival_out;
  p.service_out = service_out;
  p.gate_out = gate_out;
  p.priority_out = priority_out;
  p.mask_out = mask_out;
  p.index_out = index_out;
  p.width = width;
  p.count_out = count_out;
  const Workspace ws = layout(B, H, Q, K);
  if (vasc) {
    VASC_REQUIRE(workspace && workspace_bytes >= ws.bytes, "workspace of %zu bytes required", ws.bytes);
    VASC_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
  }
  char *wsb = static_cast<char *>(workspace);
  p.total = vasc ? reinterpret_cast<float *>(wsb + ws.total) : nullptr;
  p.rowpair = vasc ? reinterpret_cast<float *>(wsb + ws.rowpair) : nullptr;
  p.cap = vasc ? reinterpret_cast<int32_t *>(wsb + ws.cap) : nullptr;
  p.adm = vasc ? reinterpret_cast<float *>(wsb + ws.adm) : nullptr;
  p.ia = vasc ? reinterpret_cast<float2 *>(wsb + ws.ia) : nullptr;
  p.part = vasc ? reinterpret_cast<double *>(wsb + ws.part) : nullptr;
  p.gate_part = vasc ? reinterpret_cast<double *>(wsb + ws.gate_part) : nullptr;
  p.nchunks = cdiv(Q, kChunk);
  p.counts = vasc ? reinterpret_cast<int32_t *>(wsb + ws.counts) : nullptr;
  p.flags = vasc ? reinterpret_cast<int32_t *>(wsb + ws.flags) : nullptr;

  return launch_rows(p, vasc, reinterpret_cast<hipStream_t>(stream));
}

// Scratch of vasc_select_blocks_noalloc: one copy per GPU, held for the
// process lifetime. Every kernel writes each workspace word it later reads
// within the same call (the pair counts are cleared by the head pass), so
// nothing has to start at zero and no call depends on an earlier one.
static __device__ __align__(256) char scratch[VASC_SELECT_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once resolved

// Device address of the current device's scratch, resolved with
// hipGetSymbolAddress on the first call on that device (with it current).
int scratch_for_current_device(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("vasc_select_blocks_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return VASC_ERR_HIP;
  }
  VASC_SUPPORTED(dev >= 0 && dev < kMaxDevices, "device %d outside the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("vasc_select_blocks_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return VASC_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return VASC_OK;
}

}  // namespace
}  // namespace vasc

extern "C" int vasc_select_blocks(const float *score, const float *innovation, int64_t B, int64_t H, int64_t Q,
                                  int64_t K, int32_t mode, int32_t topk, const int32_t *row_cap,
                                  const uint8_t *protected_mask, int32_t force_last, int32_t max_capacity,
                                  int32_t sink_blocks, const float *debt_in, const float *pending_arrival,
                                  const float *prev_service, float *debt_out, float *arrival_out,
                                  float *service_out, int32_t *gate_out, float *priority_out, uint8_t *mask_out,
                                  int32_t *index_out, int64_t width, int32_t *count_out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  return vasc::select_blocks_impl(score, innovation, B, H, Q, K, mode, topk, row_cap, protected_mask, force_last,
                                  max_capacity, sink_blocks, debt_in, pending_arrival, prev_service, debt_out,
                                  arrival_out, service_out, gate_out, priority_out, mask_out, index_out, width,
                                  count_out, workspace, workspace_bytes, stream);
}

extern "C" int vasc_select_blocks_noalloc(const float *score, const float *innovation, int64_t B, int64_t H,
                                          int64_t Q, int64_t K, int32_t mode, int32_t topk, const int32_t *row_cap,
                                          const uint8_t *protected_mask, int32_t force_last, int32_t max_capacity,
                                          int32_t sink_blocks, const float *debt_in, const float *pending_arrival,
                                          const float *prev_service, float *debt_out, float *arrival_out,
                                          float *service_out, int32_t *gate_out, float *priority_out,
                                          uint8_t *mask_out, int32_t *index_out, int64_t width, int32_t *count_out,
                                          void *stream) {
  using namespace vasc;
  void *ws = nullptr;
  size_t bytes = 0;
  if (mode == VASC_MODE_VASC) {
    VASC_REQUIRE(B > 0 && H > 0 && Q > 0 && K > 0, "sizes must be positive");
    VASC_SUPPORTED(K <= 8192, "K=%lld key blocks not built (built: <= 8192)", (long long)K);
    const size_t need = layout(B, H, Q, K).bytes;
    VASC_REQUIRE(need <= static_cast<size_t>(VASC_SELECT_SCRATCH_BYTES),
                 "vasc_select_blocks_noalloc: these sizes need %zu bytes of scratch, above the built maximum of "
                 "%zu (VASC_SELECT_SCRATCH_BYTES); use vasc_select_blocks with a caller workspace",
                 need, static_cast<size_t>(VASC_SELECT_SCRATCH_BYTES));
    int rc;
    if ((rc = scratch_for_current_device(&ws))) return rc;
    bytes = VASC_SELECT_SCRATCH_BYTES;
  }
  return select_blocks_impl(score, innovation, B, H, Q, K, mode, topk, row_cap, protected_mask, force_last,
                            max_capacity, sink_blocks, debt_in, pending_arrival, prev_service, debt_out, arrival_out,
                            service_out, gate_out, priority_out, mask_out, index_out, width, count_out, ws, bytes,
                            stream);
}

extern "C" int vasc_settle_terminal(const float *debt_in, const float *pending_arrival, const float *service,
                                    int64_t n, float *debt_out, void *stream) {
  using namespace vasc;
  VASC_REQUIRE(pending_arrival && service && debt_out && n > 0, "invalid arguments");
  hipLaunchKernelGGL(settle_terminal_kernel, dim3(cdiv(n, 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     debt_in, pending_arrival, service, n, debt_out);
  return check_launch("vasc_settle_terminal");
}

extern "C" int vasc_cdf_counts(const float *score, int64_t B, int64_t H, int64_t Q, int64_t K,
                               const float *thresholds, int32_t min_count, int32_t force_last, int32_t *count_out,
                               int32_t *base_out, void *stream) {
  using namespace vasc;
  VASC_REQUIRE(score && thresholds && count_out, "score, thresholds and count_out are required");
  VASC_REQUIRE(B > 0 && H > 0 && Q > 0 && K > 0, "sizes must be positive");
  VASC_SUPPORTED(K <= 8192, "K=%lld key blocks not built (built: <= 8192)", (long long)K);
  VASC_REQUIRE(min_count >= 0 && min_count <= K, "min_count %d outside [0, K]", min_count);
  VASC_REQUIRE(B * H * Q < (int64_t(1) << 31), "too many rows");
  const dim3 grid(static_cast<unsigned>(B * H * Q));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int Ki = static_cast<int>(K);
  if (K <= 256 * 16) {
    // rows of up to 4096 key blocks: the radix-sorted count
    auto kern = K <= 256 ? cdf_count_radix_kernel<1>
                : K <= 512 ? cdf_count_radix_kernel<2>
                : K <= 1024 ? cdf_count_radix_kernel<4>
                : K <= 2048 ? cdf_count_radix_kernel<8>
                : cdf_count_radix_kernel<16>;
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, score, H, Q, Ki, thresholds, min_count, force_last, count_out,
                       base_out);
    return check_launch("vasc_cdf_counts");
  }
  int n2 = 64;
  while (n2 < K) n2 <<= 1;
  hipLaunchKernelGGL(cdf_count_kernel, grid, dim3(256), static_cast<size_t>(n2) * 4, st, score, H, Q, Ki, n2,
                     thresholds, min_count, force_last, count_out, base_out);
  return check_launch("vasc_cdf_counts");
}

extern "C" int vasc_priority_order(const float *priority, const int32_t *index, const int32_t *count, int64_t width,
                                   int32_t sink, int64_t rows, int64_t K, int64_t M, int64_t *order_out,
                                   void *stream) {
  using namespace vasc;
  VASC_REQUIRE(priority && order_out, "priority and order_out are required");
  VASC_REQUIRE(!index || count, "index needs count");
  VASC_REQUIRE(rows > 0 && K > 0, "sizes must be positive");
  VASC_SUPPORTED(K <= 8192, "K=%lld key blocks not built (built: <= 8192)", (long long)K);
  VASC_REQUIRE(M >= 0 && M <= K, "M=%lld outside [0, K]", (long long)M);
  VASC_REQUIRE(!index || (sink >= 0 && width >= M + sink), "index rows of width %lld cannot hold M + sink entries",
               (long long)width);
  VASC_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
  if (M == 0) return VASC_OK;
  const OrderArgs a{priority, index, index ? count : nullptr, width, sink, rows, static_cast<int>(K),
                    static_cast<int>(M), order_out};
  return launch_order(a, reinterpret_cast<hipStream_t>(stream));
}
