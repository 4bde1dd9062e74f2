// Kernel 4: block-sparse flash attention forward for gfx950 (bf16 MFMA).
//
// Semantics follow SpargeAttn's block-sparse kernel
// (ZIP:csrc/qattn/qk_int_sv_f16_cuda_sm80.cuh:42-738): one workgroup per
// (128-row query block, head, batch) walks only the 64-key blocks named by
// its list, with a base-2 softmax and masking of keys past the end. The
// arithmetic is bf16 MFMA with fp32 accumulation instead of int8 QK^T + fp16
// PV, and the structure is CDNA4's:
//
//  * 4 waves x 32 query rows. S^T = K Q^T on v_mfma_f32_32x32x16_bf16 so a
//    lane owns one query row (lane % 32) and 32 of the 64 keys of a block.
//  * O^T = Vt P^T on the same MFMA, so P feeds the B operand straight from
//    the S^T accumulators. Vt comes from vasc_pack_v with keys permuted into
//    exactly the order the accumulators hold them.
//  * The kernel is held to 128 VGPRs so four waves share each SIMD: one
//    wave's MFMAs overlap other waves' exponentials (on gfx950 a v_exp_f32
//    costs about 2.3 FMA issue slots; at head_dim 64 the exponentials cost
//    as much VALU time as the MFMAs take).
//  * The exponent offset m only has to keep probabilities inside fp32/bf16
//    range, not equal the row max: softmax is invariant to it. m starts at
//    0 and the fast path is P = exp2(fma(S, sm_scale*log2(e), -m)) on the
//    exact fp32 logits: no max, no rescale. Each lane sums its block's bf16
//    probabilities with v_dot2 (the sum is also the normaliser); a block sum
//    above 2^64, or a running sum below 2^-60 (a row whose logits are all far
//    below 0), sends the wave through an exact path that moves m to the row
//    max and rescales O and the sum. The same path masks the keys of the
//    partial last block and of blocks outside the sequence.
//  * K and Vt tiles arrive by LDS DMA (global_load_lds_dwordx4) into a
//    double-buffered LDS tile one block ahead of the MFMAs, with a
//    16-byte-chunk xor swizzle ((row/2)%8) that spreads the rows an MFMA
//    operand read touches over all LDS banks. The DMA is issued through asm
//    without a memory clobber (the explicit waits and barriers order it), so
//    the compiler neither drains it before LDS reads nor turns the uniform
//    list reads into vector loads: the lists are read through the constant
//    address space on the scalar unit, and nothing but the DMA counts in
//    vmcnt inside the loop. Q is consumed before the loop so that its load
//    wait stays out of the loop body.
//  * The loop body runs two blocks per trip (buffers 0 and 1), so every LDS
//    operand address is a lane constant plus an immediate offset; all eight K
//    (and Vt) operand reads of a block are issued before its first product.
//  * workgroup ids are remapped so each XCD walks a contiguous range of
//    query blocks of the same head (K/V reuse in that XCD's L2).
//  * vasc_global_attn_fwd adds the layer's special-token queries, which
//    attend to every key (attention.py:8480-8484), to the same launch: their
//    workgroups take the first hardware ids, so they start first (each walks
//    every key block, about four times the work of a patch-query
//    workgroup), and they are remapped like the patch workgroups, so each
//    XCD takes the special queries of the heads whose patch queries it
//    walks and reads their K and V through the same L2.
#include "common.h"

namespace vasc {
namespace {

constexpr int kBlockQ = 128;
constexpr int kBlockK = 64;
constexpr int kHeadDim = 64;
constexpr int kThreads = 256;
constexpr int kTile = kBlockK * kHeadDim;  // elements of one K or Vt tile

struct AttnParams {
  const uint16_t *q;
  int64_t q_sb, q_sh, q_st;
  const uint16_t *k;
  int64_t k_sb, k_sh, k_st;
  const uint16_t *vt;
  uint16_t *o;
  int64_t o_sb, o_sh, o_st;
  int64_t H, nq, nk, nqb, nkb;
  const int32_t *idx;
  int64_t idx_w;
  const int32_t *cnt;
  int32_t delta;
  float c;  // sm_scale * log2(e)
  int64_t num_wg;
  // special-token queries (dense over every key block), NULL when absent
  const uint16_t *q2;
  int64_t q2_sb, q2_sh, q2_st;
  uint16_t *o2;
  int64_t o2_sb, o2_sh, o2_st;
  int64_t nq2, nq2b, num_wg2, num_wg2_slots;
  // token-major output (tok_p > 0): query rows land on the frame-major token
  // rows of o (frames of tok_p tokens, tok_s special ones first)
  int64_t tok_p, tok_s;
  // 1: workgroups in hardware order, head-major (sequences whose K and V of
  // eight heads, one per XCD, would overflow the Infinity Cache); 0: each
  // XCD walks a contiguous range of query blocks
  int32_t head_major;
  // PV post-cut (kPv instances): per-head thresholds in log2 units and the
  // per-wave execution map [B, H, nqb * 4, pv_w] (written where PV ran)
  const float *pv_thr;
  int32_t *pv_map;
  int64_t pv_w;
};

__device__ __forceinline__ floatx16 mfma32(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Sum of a packed bf16 pair added to acc (v_dot2c_f32_bf16 with (1, 1)).
__device__ __forceinline__ float add_bf16_pair(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                         __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
}

// LDS chunk swizzle of tile row r (16-byte chunks, 8 per 128-byte row).
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// Exact-path triggers: a lane's block sum above kHigh (a probability may be
// near overflow) or a running sum below kLow (the row's logits are so far
// below m that they lose precision).
constexpr float kHigh = 18446744073709551616.0f;  // 2^64
constexpr float kLow = 8.673617379884035e-19f;    // 2^-60

// LDS DMA without a memory clobber (the waits and barriers that order it are
// explicit); uniform list reads then stay on the scalar unit.
__device__ __forceinline__ void dma16(const void *sbase, uint32_t voff_bytes, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(voff_bytes), "s"(sbase));
}

template <bool kDense, bool kPv = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void bsattn_fwd_kernel(const AttnParams p) {
  constexpr int CH = 512 / kThreads;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][2][kTile];  // [buffer][K, Vt]
  __shared__ float pv_gap[kPv ? 4 : 1];                                 // per-wave gap of the PV post-cut
  auto lds_u32 = [](const uint16_t *ptr) { return lds_addr32(ptr); };

  // Workgroups [0, num_wg2_slots) take the special-token queries (every key
  // block; the slot count is rounded up to a multiple of the 8 XCDs so that
  // both ranges start on XCD 0); the rest the patch queries of their lists.
  const bool dense = kDense || static_cast<int64_t>(blockIdx.x) < p.num_wg2_slots;
  const int64_t nqb = dense && !kDense ? p.nq2b : p.nqb;
  const int64_t hw = dense && !kDense ? static_cast<int64_t>(blockIdx.x)
                                      : static_cast<int64_t>(blockIdx.x) - p.num_wg2_slots;
  const int64_t wg = p.head_major ? hw : xcd_remap(hw, dense && !kDense ? p.num_wg2_slots : p.num_wg);
  if (dense && !kDense && wg >= p.num_wg2) return;  // padding of the special-query slots
  const int qb = static_cast<int>(wg % nqb);
  const int64_t bh = wg / nqb;
  const int64_t h = bh % p.H;
  const int64_t b = bh / p.H;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform
  const int l = tid & 63, lr = l & 31, hf = l >> 5;

  int n;
  const int32_t *list = nullptr;
  if (dense) {
    n = static_cast<int>(p.nkb);
  } else {
    const int64_t row = bh * p.nqb + qb;
    list = p.idx + row * p.idx_w;
    n = p.cnt[row];
    n = n < 0 ? 0 : (n > p.idx_w ? static_cast<int>(p.idx_w) : n);
  }

  const bool sp = dense && !kDense;  // a special-query workgroup
  const uint16_t *qsrc = sp ? p.q2 : p.q;
  const int64_t q_sb = sp ? p.q2_sb : p.q_sb, q_sh = sp ? p.q2_sh : p.q_sh, q_st = sp ? p.q2_st : p.q_st;
  const int64_t nq = sp ? p.nq2 : p.nq;
  uint16_t *odst = sp ? p.o2 : p.o;
  const int64_t o_sb = sp ? p.o2_sb : p.o_sb, o_sh = sp ? p.o2_sh : p.o_sh, o_st = sp ? p.o2_st : p.o_st;
  const int64_t qrow = static_cast<int64_t>(qb) * kBlockQ + w * 32 + lr;
  const bool qvalid = qrow < nq;
  // a wave whose 32 rows all lie past the queries (the short last block of
  // the special queries) only stages its share of the tiles
  const bool idle = static_cast<int64_t>(qb) * kBlockQ + w * 32 >= nq;
  int64_t orow = qvalid ? qrow : 0;
  if (p.tok_p > 0) {
    const int64_t per = sp ? p.tok_s : p.tok_p - p.tok_s;  // queries per frame of this kind
    orow = (orow / per) * p.tok_p + (sp ? 0 : p.tok_s) + orow % per;
  }
  uint16_t *optr = odst + b * o_sb + h * o_sh + orow * o_st;

  if (n == 0) {
    if (qvalid) {
#pragma unroll
      for (int c = hf; c < 8; c += 2) *reinterpret_cast<u32x4 *>(optr + c * 8) = u32x4{0, 0, 0, 0};
    }
    return;
  }

  // Q as the B operand of S^T = K Q^T: lane holds row lr, d = 16s + 8hf .. +7.
  u32x4 qf[4];
  {
    const uint16_t *qptr = qsrc + b * q_sb + h * q_sh + (qvalid ? qrow : 0) * q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[s] = qvalid ? *reinterpret_cast<const u32x4 *>(qptr + 16 * s + 8 * hf) : u32x4{0, 0, 0, 0};
    // consume Q here so that the compiler's wait for these loads lands before
    // the loop instead of inside it
    asm volatile("" ::"v"(qf[0]), "v"(qf[1]), "v"(qf[2]), "v"(qf[3]));
  }

  // Staging: LDS chunk ci = u*256 + tid lands at byte 16*ci (the DMA writes
  // lane i of a wave at base + 16*i); it holds tile row ci/8, logical chunk
  // (ci%8) ^ swz(row), so each lane fetches that global chunk.
  const uint16_t *kbase = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t *vbase = p.vt + (bh * p.nkb) * kTile;
  const int nk32 = static_cast<int>(p.nk);
  const int nkb32 = static_cast<int>(p.nkb);
  const int partial = (nk32 % kBlockK) ? nkb32 - 1 : -1;  // the partial last block, if any
  // swz(32u + r) = swz(r): a thread's chunk column, and so its byte offset
  // inside the block, is the same for each of its CH chunks; only the row
  // base (32u rows) moves, and that goes into the scalar base address.
  const int r0 = tid >> 3;
  const int cc = (tid & 7) ^ swz(r0);
  const uint32_t koff = static_cast<uint32_t>((static_cast<int64_t>(r0) * p.k_st + cc * 8) * 2);
  const uint32_t voff = static_cast<uint32_t>((r0 * kHeadDim + cc * 8) * 2);
  const int last_row = partial >= 0 ? nk32 - 1 - partial * kBlockK : kBlockK - 1;
  // K and Vt of block blk -> LDS buffer buf. Blocks outside [0, nkb) load
  // block 0 (their scores are masked); rows of the partial block past the
  // sequence end read its last row.
  auto fetch = [&](int blk, int buf) {
    const int sb = (blk >= 0 && blk < nkb32) ? blk : 0;
    const uint16_t *kb = kbase + static_cast<int64_t>(sb) * kBlockK * p.k_st;
    const uint16_t *vb = vbase + static_cast<int64_t>(sb) * kTile;
    const uint32_t kd = lds_u32(smem[buf][0]) + w * 64 * 16, vd = lds_u32(smem[buf][1]) + w * 64 * 16;
    if (sb == partial) {
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int r = 32 * u + r0;
        const int rr = r < last_row ? r : last_row;
        dma16(kb, static_cast<uint32_t>((static_cast<int64_t>(rr) * p.k_st + cc * 8) * 2), kd + u * kThreads * 16);
      }
    } else {
#pragma unroll
      for (int u = 0; u < CH; ++u) dma16(kb + 32 * u * p.k_st, koff, kd + u * kThreads * 16);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) dma16(vb + 32 * u * kHeadDim, voff, vd + u * kThreads * 16);
  };
  // Keys of block blk that exist: 64, fewer for the partial last block, 0
  // for blocks outside [0, nkb).
  auto valid_keys = [&](int blk) {
    return (blk >= 0 && blk < nkb32) ? (blk == partial ? nk32 - blk * kBlockK : kBlockK) : 0;
  };

  const floatx16 zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  floatx16 oacc[2] = {zero16, zero16};
  float ls = 0.f;  // running sum of the bf16 probabilities (this lane's 32 keys per block)
  float m = 0.f;   // exponent offset of this lane's row (log2 units)
  const float c = p.c;
  float run_max = -5000000.0f;  // PV post-cut: running row max (log2 units)
  const float pv_threshold = kPv ? p.pv_thr[h] : 0.f;

  // P = exp2(c S - m) for k-step s of the PV product (accumulators
  // 8(s%2)..+7 of tile s/2), packed to bf16; returns bs plus the sum of the
  // rounded pairs.
  auto exp_step = [&](const floatx16 (&S)[2], u32x4 (&pb)[4], int s, float bs) {
    const int t = s >> 1, r = 8 * (s & 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x0 = __builtin_amdgcn_exp2f(fmaf(S[t][r + 2 * e], c, -m));
      const float x1 = __builtin_amdgcn_exp2f(fmaf(S[t][r + 2 * e + 1], c, -m));
      pb[s][e] = pack_bf16x2(x0, x1);
      bs = add_bf16_pair(pb[s][e], bs);
    }
    return bs;
  };
  auto exp_block = [&](const floatx16 (&S)[2], u32x4 (&pb)[4]) {
    float bs0 = 0.f, bs1 = 0.f;  // two partial sums: shorter dependency chains
#pragma unroll
    for (int s = 0; s < 4; s += 2) {
      bs0 = exp_step(S, pb, s, bs0);
      bs1 = exp_step(S, pb, s + 1, bs1);
    }
    return bs0 + bs1;
  };
  // Scores of keys at or past lim (of the block's 64) to -inf. An opaque
  // copy of the lane's key offset keeps the 32 per-element key indices from
  // being hoisted out of the loop.
  auto mask_keys = [&](floatx16 (&S)[2], int lim) {
    int h4 = 4 * hf;
    asm volatile("" : "+v"(h4));
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 32 * t + 8 * (r >> 2) + h4 + (r & 3);
        S[t][r] = kk < lim ? S[t][r] : -INFINITY;
      }
  };
  // Slow path for the current block (its missing keys already masked): move m to
  // the row max where the block left the fast path's range (both lanes of a
  // row agree), rescale O and the sum, redo P. Rows whose running sum is
  // negligible drop it (it holds no information relative to the new m)
  // instead of scaling it up.
  auto slow = [&](floatx16 (&S)[2], u32x4 (&pb)[4]) {
    float mx = S[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, S[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[1][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    mx = mx == -INFINITY ? mx : mx * c - m;  // block max relative to m, log2 units
    const float lrow = ls + __shfl_xor(ls, 32);
    const bool tiny = !(lrow >= kLow);
    // g: how far m moves. Up to the block max when it is above m; down to it
    // only when the row so far is negligible (or empty).
    float g = 0.f;
    if (mx != -INFINITY) g = (mx > 0.f || tiny) ? mx : 0.f;
    const float alpha = tiny ? 0.f : __builtin_amdgcn_exp2f(-g);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      oacc[0][r] *= alpha;
      oacc[1][r] *= alpha;
    }
    ls *= alpha;
    m += g;
    return exp_block(S, pb);
  };

  // List entry j+1 is loaded during iteration j-1 (index clamped to the list)
  // so that reading it never waits on memory: the wait at the top of each
  // iteration already covers it.
  const __attribute__((address_space(4))) int32_t *clist =
      (const __attribute__((address_space(4))) int32_t *)(list);
  int blk = dense ? 0 : clist[0];
  int32_t e_next = dense ? 0 : clist[n > 1 ? 1 : 0];
  fetch(blk, 0);
  // One block: wait for its tiles, start the next block's DMA into the other
  // buffer, compute. The loop runs two blocks per trip so that each block's
  // buffer, and with it every LDS address, is a compile-time constant.
  auto step = [&](const int j, const int buf) {
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    const int cur = blk;
    if (j + 1 < n) {
      if (dense) {
        blk = j + 1;
      } else {
        const int e = e_next;
        blk = p.delta ? blk + e : e;
        e_next = clist[j + 2 < n ? j + 2 : n - 1];
      }
      fetch(blk, buf ^ 1);
    }
    const uint16_t *ks = smem[buf][0];
    const uint16_t *vs = smem[buf][1];
    if (!kPv && idle) return;

    // S^T tiles: keys 32t + [0,32) x this wave's 32 query rows.
    floatx16 S[2];
    u32x4 ka[4][2];  // all K operands of the block, read before the first product
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 32 * t + lr;
        ka[s][t] = *reinterpret_cast<const u32x4 *>(ks + row * kHeadDim + ((2 * s + hf) ^ swz(row)) * 8);
      }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) S[t] = mfma32(ka[s][t], qf[s], s == 0 ? zero16 : S[t]);
    // every K read issued before the first score product
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);

    // PV post-cut (qk_int_sv_f16_cuda_sm80.cuh:291-381 with update_mo,
    // attn_utils.cuh:419-466, per-block mode): gap = the largest over the
    // workgroup's rows of (block row max - running max) in log2 units; the
    // running max starts at -5e6 and follows every listed block, executed or
    // not; PV runs for the whole workgroup only when gap + threshold > 0.
    if constexpr (kPv) {
      if (!dense) {
        const int lim = valid_keys(cur);
        float mx = -5000000.0f;
        if (lim == kBlockK) {  // a whole block (the usual case): no per-key masks
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[t][r]);
        } else {
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kk = 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
              mx = kk < lim ? fmaxf(mx, S[t][r]) : mx;
            }
        }
        mx = fmaxf(mx, xor_lane(mx, 32)) * c;
        float gap = mx - run_max;  // the wave's largest, by VALU cross-lane moves (rows 0-31, both halves)
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) gap = fmaxf(gap, xor_lane(gap, off));
        run_max = fmaxf(run_max, mx);
        if (l == 0) pv_gap[w] = gap;
      }
    }

    // keys past the sequence end (partial or out-of-range blocks) are masked
    // before the exponentials, so such a block stays on the fast path unless
    // its sums leave the range
    const int lim = valid_keys(cur);
    if (lim < kBlockK) mask_keys(S, lim);
    u32x4 pb[4];
    float bs = exp_block(S, pb);  // changes no state: a skipped block drops it
    if constexpr (kPv) {
      if (!dense) {
        // the workgroup's decision, read after the exponentials so that the
        // barrier wait overlaps them
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const float g4 = fmaxf(fmaxf(pv_gap[0], pv_gap[1]), fmaxf(pv_gap[2], pv_gap[3]));
        if (!(g4 + pv_threshold > 0.f)) return;  // skipped: no sum, no PV
        if (l == 0 && p.pv_map && cur >= 0 && cur < nkb32)
          p.pv_map[((bh * p.nqb + qb) * 4 + w) * p.pv_w + cur] = 1;
      }
    }
    if (__ballot(!(bs <= kHigh) || !(ls + bs >= kLow))) bs = slow(S, pb);
    ls += bs;

    u32x4 va[4][2];  // all Vt operands of the block, read before the first product
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        const int row = 32 * n2 + lr;
        va[s][n2] = *reinterpret_cast<const u32x4 *>(vs + row * kHeadDim + ((2 * s + hf) ^ swz(row)) * 8);
      }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) oacc[n2] = mfma32(va[s][n2], pb[s], oacc[n2]);
    // every Vt read issued before the first PV product
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  };
  for (int j = 0; j < n; j += 2) {
    step(j, 0);
    if (j + 1 < n) step(j + 1, 1);
  }

  const float ltot = ls + __shfl_xor(ls, 32);
  const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
  if (qvalid) {
#pragma unroll
    for (int n2 = 0; n2 < 2; ++n2)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * n2 + 8 * g + 4 * hf;
        uint2 v;
        v.x = pack_bf16x2(oacc[n2][4 * g + 0] * inv, oacc[n2][4 * g + 1] * inv);
        v.y = pack_bf16x2(oacc[n2][4 * g + 2] * inv, oacc[n2][4 * g + 3] * inv);
        *reinterpret_cast<uint2 *>(optr + d0) = v;
      }
  }
}

int check_bhtd(const char *name, const void *ptr, int64_t sb, int64_t sh, int64_t st) {
  VASC_REQUIRE(ptr != nullptr, "%s is NULL", name);
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(ptr) & 15) == 0, "%s must be 16-byte aligned", name);
  VASC_REQUIRE(sb % 8 == 0 && sh % 8 == 0 && st % 8 == 0 && sb >= 0 && sh >= 0 && st > 0,
               "%s strides (%lld,%lld,%lld) must be non-negative multiples of 8 elements", name,
               (long long)sb, (long long)sh, (long long)st);
  return VASC_OK;
}

// Token-major output of vasc_global_attn_tokens_fwd (absent: P == 0).
struct OutTokens {
  int64_t P = 0, S = 0;
};

// Special-token queries of vasc_global_attn_fwd (absent: q2 == NULL).
struct SpecialQueries {
  const uint16_t *q2 = nullptr;
  int64_t q2_sb = 0, q2_sh = 0, q2_st = 0;
  uint16_t *o2 = nullptr;
  int64_t o2_sb = 0, o2_sh = 0, o2_st = 0;
  int64_t nq2 = 0;
};

int launch_attn(bool dense, const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st, const uint16_t *vt,
                uint16_t *o, int64_t o_sb, int64_t o_sh, int64_t o_st, int64_t B, int64_t H,
                int64_t nq, int64_t nk, int64_t d, const int32_t *idx, int64_t idx_w,
                const int32_t *cnt, int32_t delta, float sm_scale, void *stream,
                const SpecialQueries &sq = SpecialQueries(), const float *pv_thr = nullptr,
                int32_t *pv_map = nullptr, const OutTokens &ot = OutTokens()) {
  VASC_SUPPORTED(d == kHeadDim, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(B > 0 && H > 0 && nq > 0 && nk > 0, "sizes must be positive");
  int rc;
  if ((rc = check_bhtd("q", q, q_sb, q_sh, q_st))) return rc;
  if ((rc = check_bhtd("k", k, k_sb, k_sh, k_st))) return rc;
  if ((rc = check_bhtd("o", o, o_sb, o_sh, o_st))) return rc;
  VASC_REQUIRE(vt != nullptr && (reinterpret_cast<uintptr_t>(vt) & 15) == 0, "vt must be a 16-byte aligned packed V");
  if (!dense) {
    VASC_REQUIRE(idx != nullptr && cnt != nullptr, "block_index and block_count are required");
    VASC_REQUIRE(idx_w > 0, "index_width must be positive");
  }
  VASC_REQUIRE(sm_scale > 0.f, "sm_scale must be positive");
  AttnParams p;
  p.q = q; p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.k = k; p.k_sb = k_sb; p.k_sh = k_sh; p.k_st = k_st;
  p.vt = vt;
  p.o = o; p.o_sb = o_sb; p.o_sh = o_sh; p.o_st = o_st;
  p.H = H; p.nq = nq; p.nk = nk;
  p.nqb = cdiv(nq, kBlockQ);
  p.nkb = cdiv(nk, kBlockK);
  p.idx = idx; p.idx_w = idx_w; p.cnt = cnt; p.delta = delta;
  p.c = sm_scale * 1.4426950408889634f;
  p.num_wg = B * H * p.nqb;
  p.q2 = sq.q2; p.q2_sb = sq.q2_sb; p.q2_sh = sq.q2_sh; p.q2_st = sq.q2_st;
  p.o2 = sq.o2; p.o2_sb = sq.o2_sb; p.o2_sh = sq.o2_sh; p.o2_st = sq.o2_st;
  p.nq2 = sq.q2 ? sq.nq2 : 0;
  p.nq2b = cdiv(p.nq2, kBlockQ);
  p.num_wg2 = B * H * p.nq2b;
  p.num_wg2_slots = (p.num_wg2 + 7) / 8 * 8;
  // K and V of one head take 256 B per key token; from 192k tokens (48 MB a
  // head) the eight heads one per XCD that the contiguous mapping keeps in
  // flight exceed the 256 MB Infinity Cache by half, and walking the heads
  // one after another across all XCDs reads less from HBM (7 % faster at
  // 256k tokens, no change at 133k, 2 % slower at C2)
  p.head_major = nk >= 192 * 1024 ? 1 : 0;
  VASC_REQUIRE(p.num_wg + p.num_wg2_slots < (int64_t(1) << 31), "grid too large");
  VASC_SUPPORTED(nk < (int64_t(1) << 30) && nq < (int64_t(1) << 40), "sequence of %lld keys not built (< 2^30)",
                 (long long)nk);
  p.pv_thr = pv_thr;
  p.pv_map = pv_map;
  p.pv_w = p.nkb;
  p.tok_p = ot.P;
  p.tok_s = ot.S;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto kern = dense ? bsattn_fwd_kernel<true> : (pv_thr ? bsattn_fwd_kernel<false, true> : bsattn_fwd_kernel<false>);
  hipLaunchKernelGGL(kern, dim3(p.num_wg + p.num_wg2_slots), dim3(kThreads), 0, s, p);
  return check_launch(dense ? "vasc_dense_attn_fwd" : "vasc_block_sparse_attn_fwd");
}

}  // namespace
}  // namespace vasc

extern "C" int vasc_block_sparse_attn_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                          const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                          const uint16_t *vt, uint16_t *o, int64_t o_sb, int64_t o_sh,
                                          int64_t o_st, int64_t B, int64_t H, int64_t nq, int64_t nk,
                                          int64_t d, const int32_t *block_index, int64_t index_width,
                                          const int32_t *block_count, int32_t index_is_delta,
                                          float sm_scale, void *stream) {
  return vasc::launch_attn(false, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, vt, o, o_sb, o_sh, o_st, B, H,
                           nq, nk, d, block_index, index_width, block_count, index_is_delta, sm_scale,
                           stream);
}

extern "C" int vasc_block_sparse_attn_pv_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                             const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                             const uint16_t *vt, uint16_t *o, int64_t o_sb, int64_t o_sh,
                                             int64_t o_st, int64_t B, int64_t H, int64_t nq, int64_t nk,
                                             int64_t d, const int32_t *block_index, int64_t index_width,
                                             const int32_t *block_count, int32_t index_is_delta, float sm_scale,
                                             const float *pv_threshold, int32_t *pv_map, void *stream) {
  VASC_REQUIRE(pv_threshold != nullptr, "pv_threshold ([H] float32, device) is required");
  return vasc::launch_attn(false, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, vt, o, o_sb, o_sh, o_st, B, H,
                           nq, nk, d, block_index, index_width, block_count, index_is_delta, sm_scale, stream,
                           vasc::SpecialQueries(), pv_threshold, pv_map);
}

extern "C" int vasc_dense_attn_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                   const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                   const uint16_t *vt, uint16_t *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                                   int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d, float sm_scale,
                                   void *stream) {
  return vasc::launch_attn(true, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, vt, o, o_sb, o_sh, o_st, B, H, nq,
                           nk, d, nullptr, 1, nullptr, 0, sm_scale, stream);
}

extern "C" int vasc_global_attn_fwd(const uint16_t *q_patch, int64_t qp_sb, int64_t qp_sh, int64_t qp_st,
                                    const uint16_t *q_special, int64_t qs_sb, int64_t qs_sh, int64_t qs_st,
                                    const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                    const uint16_t *vt, uint16_t *o_patch, int64_t op_sb, int64_t op_sh,
                                    int64_t op_st, uint16_t *o_special, int64_t os_sb, int64_t os_sh,
                                    int64_t os_st, int64_t B, int64_t H, int64_t n_patch, int64_t n_special,
                                    int64_t nk, int64_t d, const int32_t *block_index, int64_t index_width,
                                    const int32_t *block_count, float sm_scale, void *stream) {
  using namespace vasc;
  SpecialQueries sq;
  if (n_special > 0) {
    int rc;
    if ((rc = check_bhtd("q_special", q_special, qs_sb, qs_sh, qs_st))) return rc;
    if ((rc = check_bhtd("o_special", o_special, os_sb, os_sh, os_st))) return rc;
    sq.q2 = q_special; sq.q2_sb = qs_sb; sq.q2_sh = qs_sh; sq.q2_st = qs_st;
    sq.o2 = o_special; sq.o2_sb = os_sb; sq.o2_sh = os_sh; sq.o2_st = os_st;
    sq.nq2 = n_special;
  }
  VASC_REQUIRE(n_special >= 0, "n_special must be non-negative");
  return launch_attn(false, q_patch, qp_sb, qp_sh, qp_st, k, k_sb, k_sh, k_st, vt, o_patch, op_sb, op_sh, op_st,
                     B, H, n_patch, nk, d, block_index, index_width, block_count, 0, sm_scale, stream, sq);
}

extern "C" int vasc_global_attn_tokens_fwd(const uint16_t *q_patch, int64_t qp_sb, int64_t qp_sh, int64_t qp_st,
                                           const uint16_t *q_special, int64_t qs_sb, int64_t qs_sh, int64_t qs_st,
                                           const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                           const uint16_t *vt, uint16_t *out, int64_t B, int64_t H, int64_t N,
                                           int64_t P, int64_t S, int64_t nk, int64_t d,
                                           const int32_t *block_index, int64_t index_width,
                                           const int32_t *block_count, float sm_scale, void *stream) {
  using namespace vasc;
  VASC_REQUIRE(N > 0 && P > S && S >= 0, "invalid frame sizes N=%lld P=%lld S=%lld", (long long)N, (long long)P,
               (long long)S);
  VASC_REQUIRE(nk == N * P, "nk %lld must be N*P = %lld", (long long)nk, (long long)(N * P));
  VASC_REQUIRE(out != nullptr && (reinterpret_cast<uintptr_t>(out) & 15) == 0, "out must be a 16-byte aligned [B,N*P,H*d]");
  // out [B, N*P, H*d] contiguous: (b, h, token) strides
  const int64_t o_sb = N * P * H * d, o_sh = d, o_st = H * d;
  SpecialQueries sq;
  if (S > 0) {
    int rc;
    if ((rc = check_bhtd("q_special", q_special, qs_sb, qs_sh, qs_st))) return rc;
    sq.q2 = q_special; sq.q2_sb = qs_sb; sq.q2_sh = qs_sh; sq.q2_st = qs_st;
    sq.o2 = out; sq.o2_sb = o_sb; sq.o2_sh = o_sh; sq.o2_st = o_st;
    sq.nq2 = N * S;
  }
  OutTokens ot;
  ot.P = P;
  ot.S = S;
  return launch_attn(false, q_patch, qp_sb, qp_sh, qp_st, k, k_sb, k_sh, k_st, vt, out, o_sb, o_sh, o_st, B, H,
                     N * (P - S), nk, d, block_index, index_width, block_count, 0, sm_scale, stream, sq, nullptr,
                     nullptr, ot);
}
