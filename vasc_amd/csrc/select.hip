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
// own (contraction is off for this file) and every sum uses one of two
// canonical float64 orders, shared with the CPU oracle:
//   wave sum  lane j adds elements j, j+64, ... in order, then an xor
//             butterfly over offsets 32..1;
//   seq sum   strictly sequential in index order;
//   chunked   seq sums of consecutive 32-element chunks, then a seq sum of
//             the chunk partials (the arrival mean over query rows);
//   global    wave sum per head, then a seq sum over heads (the gate).
// Selection keeps the c largest priorities, ties to the lower block index.
//
// Launches (VASC mode): arrival (one wave per row) -> colsum (one thread per
// pair column and 32-row chunk) -> head (ledger settlement, arrival mean,
// admitted debt; one thread per pair column) -> select (one wave per row,
// radix select on order-preserving uint32 keys staged in LDS) -> service.
// Top-K mode runs the select launch alone. Every launch is short and wide:
// no long serial chains.
#pragma clang fp contract(off)

#include "common.h"

namespace vasc {
namespace {

constexpr float kFltMax = 3.402823466e38f;
constexpr float kFltMin = 1.175494351e-38f;
constexpr int kRowsPerWg = 4;   // select: one row per wave, 4 rows of one head
constexpr int kChunk = 32;      // rows per partial of the arrival mean

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
  float *total, *rowpair, *a, *adm;
  double *part, *gate_part;
  int32_t *cap, *counts;
  int64_t nchunks;
};

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

// Global service gate (sparse_wrapper.py:3837-3842) from the per-head
// partials; every caller recomputes the same bits.
__device__ __forceinline__ int service_gate(const SelectParams &p) {
  if (!p.pending) return 0;
  double u = 0.0, w = 0.0, c = 0.0;
  for (int64_t h = 0; h < p.BH; ++h) {
    u = u + p.gate_part[3 * h + 0];
    w = w + p.gate_part[3 * h + 1];
    c = c + p.gate_part[3 * h + 2];
  }
  const float fu = static_cast<float>(u), fw = static_cast<float>(w), fc = static_cast<float>(c);
  return (fc > 0.f) && (fu >= fw);
}

// ------------------------------------------------------------------ arrival
// Per-row capacity when it is not given: max(topk,1), plus one when the
// forced mixed-tail block is not already among the top-k scores (the base
// map's row count, sparse_wrapper.py:7592-7604).
__device__ int derived_cap(const SelectParams &p, const float *srow, int lane) {
  int t = p.topk < 1 ? 1 : p.topk;
  if (t > p.K) t = static_cast<int>(p.K);
  if (!p.force_last || t >= p.K) return t;
  const uint32_t last = order_key(srow[p.K - 1]);
  int beat = 0;
  for (int64_t k = lane; k < p.K; k += 64) {
    const uint32_t key = order_key(srow[k]);
    beat += (key > last) || (key == last && k < p.K - 1);
  }
  beat = wave_sum_int(beat);
  return t + (beat >= t ? 1 : 0);
}

__global__ __launch_bounds__(256) void arrival_kernel(const SelectParams p) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= p.BH * p.Q) return;
  const int lane = threadIdx.x & 63;
  const int64_t bh = row / p.Q;
  const float *srow = p.score + row * p.K;
  const float *iota = p.innovation + bh * p.P;
  const int cap = p.row_cap ? p.row_cap[row] : derived_cap(p, srow, lane);

  double acc = 0.0;
  for (int64_t k = lane; k < p.K; k += 64) acc = acc + static_cast<double>(clean_score(srow[k]) * iota[k >> 1]);
  const float total = static_cast<float>(wave_butterfly(acc));
  const float scale = static_cast<float>(cap) / floor_tiny(total);

  double racc = 0.0;
  float *arow = p.a + row * p.P;
  for (int64_t base = 0; base < p.K; base += 64) {
    const int64_t k = base + lane;
    float A = 0.f;
    if (k < p.K && total > 0.f) A = clamp01((clean_score(srow[k]) * iota[k >> 1]) * scale);
    const float An = __shfl_down(A, 1);
    if (k < p.K && (lane & 1) == 0) {
      const float ap = (k + 1 < p.K) ? (A + An) / 2.0f : (A + 0.0f) / 1.0f;
      arow[k >> 1] = ap;
      racc = racc + static_cast<double>(ap);
    }
  }
  const float rowpair = static_cast<float>(wave_butterfly(racc));
  if (lane == 0) {
    p.total[row] = total;
    p.rowpair[row] = rowpair;
    p.cap[row] = cap;
  }
}

// ------------------------------------------------------------------ head
// Partial column sums of the row pair arrival over 32-row chunks.
__global__ __launch_bounds__(256) void colsum_kernel(const SelectParams p) {
  const int64_t pp = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t chunk = blockIdx.y, bh = blockIdx.z;
  if (pp >= p.P) return;
  const int64_t q0 = chunk * kChunk;
  const int64_t q1 = q0 + kChunk < p.Q ? q0 + kChunk : p.Q;
  const float *col = p.a + (bh * p.Q) * p.P + pp;
  float v[kChunk];
#pragma unroll
  for (int i = 0; i < kChunk; ++i) v[i] = (q0 + i < q1) ? col[(q0 + i) * p.P] : 0.f;
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < kChunk; ++i)
    if (q0 + i < q1) acc = acc + static_cast<double>(v[i]);
  p.part[(bh * p.nchunks + chunk) * p.P + pp] = acc;
}

// Per head: ledger settlement, pending arrival (mean over rows), pair
// capacity and admitted debt. Wave 0 of every workgroup recomputes the head's
// debt sum and pair capacity (canonical wave sums); workgroup 0 of the head
// also publishes the head's partials of the three global gate sums.
__global__ __launch_bounds__(256) void head_kernel(const SelectParams p) {
  __shared__ float sh_pc, sh_dsum;
  const int64_t bh = blockIdx.y;
  const int tid = threadIdx.x;
  if (tid < 64) {
    double acc = 0.0, dacc = 0.0, useful = 0.0, wasted = 0.0, consumed = 0.0;
    for (int64_t q = tid; q < p.Q; q += 64) acc = acc + static_cast<double>(p.rowpair[bh * p.Q + q]);
    for (int64_t pp = tid; pp < p.P; pp += 64) {
      float refl, sig;
      const float d = settle_one(p, bh * p.P + pp, &refl, &sig);
      dacc = dacc + static_cast<double>(d);
      useful = useful + static_cast<double>(clamp_min0(sig - refl));
      wasted = wasted + static_cast<double>(refl);
      consumed = consumed + static_cast<double>(sig);
    }
    const double s = wave_butterfly(acc);
    const double ds = wave_butterfly(dacc);
    useful = wave_butterfly(useful);
    wasted = wave_butterfly(wasted);
    consumed = wave_butterfly(consumed);
    if (tid == 0) {
      sh_pc = static_cast<float>(s / static_cast<double>(p.Q));
      sh_dsum = static_cast<float>(ds);
      if (blockIdx.x == 0) {
        p.gate_part[3 * bh + 0] = useful;
        p.gate_part[3 * bh + 1] = wasted;
        p.gate_part[3 * bh + 2] = consumed;
      }
    }
  }
  __syncthreads();
  const int64_t pp = static_cast<int64_t>(blockIdx.x) * 256 + tid;
  if (pp >= p.P) return;
  double acc = 0.0;
  const double *part = p.part + bh * p.nchunks * p.P + pp;
#pragma unroll 8
  for (int64_t c = 0; c < p.nchunks; ++c) acc = acc + part[c * p.P];
  p.arrival_out[bh * p.P + pp] = static_cast<float>(acc / static_cast<double>(p.Q));
  p.counts[bh * p.P + pp] = 0;
  float refl, sig;
  const float d = settle_one(p, bh * p.P + pp, &refl, &sig);
  p.debt_out[bh * p.P + pp] = d;
  const float dsum = sh_dsum;
  const float scale = sh_pc / floor_tiny(dsum);
  p.adm[bh * p.P + pp] = dsum > 0.f ? clamp01(d * scale) : 0.f;
}

// ------------------------------------------------------------------ select
// Wave-level radix select: returns the key T of the c-th largest element
// (1 <= c <= K) and, through need, how many elements equal to T to keep.
__device__ uint32_t radix_threshold(const uint32_t *keys, int64_t K, uint32_t *hist, int lane, int &need) {
  uint32_t prefix = 0, pmask = 0;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
#pragma unroll
    for (int i = 0; i < 4; ++i) hist[4 * lane + i] = 0;
    wave_sync();
    for (int64_t k = lane; k < K; k += 64) {
      const uint32_t key = keys[k];
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    wave_sync();
    const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
    const int v = static_cast<int>(h0 + h1 + h2 + h3);
    int suf = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_down(suf, off);
      if (lane + off < 64) suf += t;
    }
    const uint64_t ball = __ballot(suf >= need);
    const int L = 63 - __clzll(static_cast<long long>(ball));
    int above = __shfl(suf - v, L);
    int digit = 0, above_l = above;
    if (lane == L) {
      const uint32_t hs[4] = {h0, h1, h2, h3};
      digit = 4 * L;
      for (int b = 3; b >= 0; --b) {
        if (above_l + static_cast<int>(hs[b]) >= need) {
          digit = 4 * L + b;
          break;
        }
        above_l += static_cast<int>(hs[b]);
      }
    }
    digit = __shfl(digit, L);
    above = __shfl(above_l, L);
    need -= above;
    prefix |= static_cast<uint32_t>(digit) << shift;
    pmask |= 0xffu << shift;
    wave_sync();
  }
  return prefix;
}

__global__ __launch_bounds__(256) void select_kernel(const SelectParams p) {
  extern __shared__ uint32_t lds[];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int64_t bh = blockIdx.y;
  const bool vasc = p.mode == VASC_MODE_VASC;
  uint32_t *keys = lds + static_cast<int64_t>(w) * p.K;
  uint32_t *hist = lds + 4 * p.K + 256 * w;
  uint32_t *pair_cnt = lds + 4 * p.K + 1024;
  if (vasc) {
    for (int64_t i = tid; i < p.P; i += 256) pair_cnt[i] = 0;
    __syncthreads();
  }
  const int gate = vasc ? service_gate(p) : 0;
  const float *iota = vasc ? p.innovation + bh * p.P : nullptr;
  const float *adm = vasc ? p.adm + bh * p.P : nullptr;

  for (int rr = w; rr < kRowsPerWg; rr += 4) {
    const int64_t q = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + rr;
    if (q >= p.Q) break;
    const int64_t row = bh * p.Q + q;
    const float *srow = p.score + row * p.K;
    int c;
    if (vasc) {
      const int cap = p.cap[row];
      c = cap < p.max_capacity ? cap : p.max_capacity;
      const float total = p.total[row];
      const float scale = static_cast<float>(cap) / floor_tiny(total);
      for (int64_t k = lane; k < p.K; k += 64) {
        float A = 0.f;
        if (total > 0.f) A = clamp01((clean_score(srow[k]) * iota[k >> 1]) * scale);
        float prio = gate ? A + adm[k >> 1] : A;
        if ((p.protected_mask && p.protected_mask[row * p.K + k]) || (p.force_last && k == p.K - 1)) prio = kFltMax;
        if (p.priority_out) p.priority_out[row * p.K + k] = prio;
        keys[k] = order_key(prio);
      }
    } else {
      c = derived_cap(p, srow, lane);
      for (int64_t k = lane; k < p.K; k += 64) {
        uint32_t key = order_key(srow[k]);
        if (p.force_last && k == p.K - 1) key = 0xffffffffu;
        keys[k] = key;
      }
    }
    c = c < 0 ? 0 : (c > p.K ? static_cast<int>(p.K) : c);
    wave_sync();

    uint32_t T = 0;
    int need = 0;
    bool all = c >= p.K, none = c == 0;
    if (!all && !none) {
      need = c;
      T = radix_threshold(keys, p.K, hist, lane, need);
    }
    int32_t *irow = p.index_out + row * p.width;
    int run_eq = 0, run_sel = 0;
    for (int64_t base = 0; base < p.K; base += 64) {
      const int64_t k = base + lane;
      const bool valid = k < p.K;
      const uint32_t key = valid ? keys[k] : 0u;
      const bool gt = valid && (all || (!none && key > T));
      const bool eq = valid && !all && !none && key == T;
      const uint64_t beq = __ballot(eq);
      const int eq_before = run_eq + __popcll(beq & lanemask_lt());
      const bool sel = gt || (eq && eq_before < need);
      const uint64_t bsel = __ballot(sel);
      const int pos = run_sel + __popcll(bsel & lanemask_lt());
      if (sel && pos < p.width) {
        irow[pos] = static_cast<int32_t>(k);
        if (vasc) atomicAdd(&pair_cnt[k >> 1], 1u);
      }
      if (valid && p.mask_out) p.mask_out[row * p.K + k] = sel ? 1 : 0;
      run_eq += __popcll(beq);
      run_sel += __popcll(bsel);
    }
    for (int i = lane; i < p.sink && run_sel + i < p.width; i += 64) irow[run_sel + i] = static_cast<int32_t>(p.K + i);
    if (lane == 0) p.count_out[row] = run_sel + p.sink;
    wave_sync();
  }
  if (vasc) {
    __syncthreads();
    for (int64_t i = tid; i < p.P; i += 256) {
      const uint32_t v = pair_cnt[i];
      if (v) atomicAdd(&p.counts[bh * p.P + i], static_cast<int32_t>(v));
    }
  }
}

// ------------------------------------------------------------------ service
__global__ __launch_bounds__(256) void service_kernel(const SelectParams p) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= p.BH * p.P) return;
  const int64_t pp = i % p.P;
  const float pair_size = (p.K % 2 && pp == p.P - 1) ? 1.0f : 2.0f;
  const float denom = pair_size * static_cast<float>(p.Q);
  p.service_out[i] = static_cast<float>(p.counts[i]) / denom;
  if (i == 0 && p.gate_out) *p.gate_out = service_gate(p);
}

__global__ void settle_terminal_kernel(const float *debt_in, const float *pending, const float *service, int64_t n,
                                       float *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float d = debt_in ? clamp_min0(debt_in[i]) : 0.f;
  out[i] = clamp_min0((d + pending[i]) - service[i]);
}

struct Workspace {
  size_t total, rowpair, cap, a, adm, part, gate_part, counts, bytes;
};

Workspace layout(int64_t B, int64_t H, int64_t Q, int64_t K) {
  const size_t BH = static_cast<size_t>(B * H), P = static_cast<size_t>((K + 1) / 2);
  Workspace w;
  size_t off = 0;
  w.total = off;   off += align256(BH * Q * 4);
  w.rowpair = off; off += align256(BH * Q * 4);
  w.cap = off;     off += align256(BH * Q * 4);
  w.a = off;       off += align256(BH * Q * P * 4);
  w.adm = off;     off += align256(BH * P * 4);
  w.part = off;    off += align256(BH * static_cast<size_t>(cdiv(Q, kChunk)) * P * 8);
  w.gate_part = off; off += align256(BH * 3 * 8);
  w.counts = off;  off += align256(BH * P * 4);
  w.bytes = off;
  return w;
}

}  // namespace
}  // namespace vasc

extern "C" size_t vasc_select_workspace_size(int64_t B, int64_t H, int64_t q_blocks, int64_t k_blocks) {
  if (B <= 0 || H <= 0 || q_blocks <= 0 || k_blocks <= 0) return 0;
  return vasc::layout(B, H, q_blocks, k_blocks).bytes;
}

extern "C" int vasc_select_blocks(const float *score, const float *innovation, int64_t B, int64_t H, int64_t Q,
                                  int64_t K, int32_t mode, int32_t topk, const int32_t *row_cap,
                                  const uint8_t *protected_mask, int32_t force_last, int32_t max_capacity,
                                  int32_t sink_blocks, const float *debt_in, const float *pending_arrival,
                                  const float *prev_service, float *debt_out, float *arrival_out,
                                  float *service_out, int32_t *gate_out, float *priority_out, uint8_t *mask_out,
                                  int32_t *index_out, int64_t width, int32_t *count_out, void *workspace,
                                  size_t workspace_bytes, void *stream) {
  using namespace vasc;
  VASC_REQUIRE(score && index_out && count_out, "score, index_out and count_out are required");
  VASC_REQUIRE(B > 0 && H > 0 && Q > 0 && K > 0, "sizes must be positive");
  VASC_SUPPORTED(K <= 8192, "K=%lld key blocks not built (built: <= 8192)", (long long)K);
  VASC_REQUIRE(mode == VASC_MODE_TOPK || mode == VASC_MODE_VASC, "unknown mode %d", mode);
  VASC_REQUIRE(sink_blocks >= 0, "sink_blocks must be non-negative");
  VASC_REQUIRE(B * H < 65536, "B*H too large");
  const bool vasc = mode == VASC_MODE_VASC;
  int64_t maxc;
  if (vasc) {
    VASC_REQUIRE(innovation && debt_out && arrival_out && service_out, "VASC needs innovation and state outputs");
    VASC_REQUIRE(max_capacity >= 0, "max_capacity must be non-negative");
    VASC_REQUIRE(!prev_service || pending_arrival, "prev_service without pending_arrival");
    maxc = max_capacity < K ? max_capacity : K;
  } else {
    int64_t t = topk < 1 ? 1 : topk;
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
  p.a = vasc ? reinterpret_cast<float *>(wsb + ws.a) : nullptr;
  p.adm = vasc ? reinterpret_cast<float *>(wsb + ws.adm) : nullptr;
  p.part = vasc ? reinterpret_cast<double *>(wsb + ws.part) : nullptr;
  p.gate_part = vasc ? reinterpret_cast<double *>(wsb + ws.gate_part) : nullptr;
  p.nchunks = cdiv(Q, kChunk);
  p.counts = vasc ? reinterpret_cast<int32_t *>(wsb + ws.counts) : nullptr;

  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t rows = p.BH * Q;
  const size_t lds = (4 * static_cast<size_t>(K) + 1024 + (vasc ? static_cast<size_t>(p.P) : 0)) * 4;
  VASC_SUPPORTED(lds <= 160 * 1024, "select needs %zu bytes of LDS", lds);
  int rc;
  if (vasc) {
    hipLaunchKernelGGL(arrival_kernel, dim3(cdiv(rows, 4)), dim3(256), 0, s, p);
    if ((rc = check_launch("vasc_select_blocks/arrival"))) return rc;
    hipLaunchKernelGGL(colsum_kernel, dim3(cdiv(p.P, 256), p.nchunks, p.BH), dim3(256), 0, s, p);
    if ((rc = check_launch("vasc_select_blocks/colsum"))) return rc;
    hipLaunchKernelGGL(head_kernel, dim3(cdiv(p.P, 256), p.BH), dim3(256), 0, s, p);
    if ((rc = check_launch("vasc_select_blocks/head"))) return rc;
  }
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(select_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) {
      set_error("vasc_select_blocks: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
      return VASC_ERR_HIP;
    }
  }
  hipLaunchKernelGGL(select_kernel, dim3(cdiv(Q, kRowsPerWg), p.BH), dim3(256), lds, s, p);
  if ((rc = check_launch("vasc_select_blocks/select"))) return rc;
  if (vasc) {
    hipLaunchKernelGGL(service_kernel, dim3(cdiv(p.BH * p.P, 256)), dim3(256), 0, s, p);
    if ((rc = check_launch("vasc_select_blocks/service"))) return rc;
  }
  return VASC_OK;
}

extern "C" int vasc_settle_terminal(const float *debt_in, const float *pending_arrival, const float *service,
                                    int64_t n, float *debt_out, void *stream) {
  using namespace vasc;
  VASC_REQUIRE(pending_arrival && service && debt_out && n > 0, "invalid arguments");
  hipLaunchKernelGGL(settle_terminal_kernel, dim3(cdiv(n, 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     debt_in, pending_arrival, service, n, debt_out);
  return check_launch("vasc_settle_terminal");
}
