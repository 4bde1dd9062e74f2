// Kernel 4: block-sparse flash attention forward for gfx950 (bf16 MFMA).
//
// Semantics follow SpargeAttn's block-sparse kernel
// (ZIP:csrc/qattn/qk_int_sv_f16_cuda_sm80.cuh:42-738): one workgroup per
// (128-row query block, head, batch) walks only the 64-key blocks named by
// its list, with an online base-2 softmax and masking of keys past the end.
// The arithmetic is bf16 MFMA with fp32 accumulation instead of int8 QK^T +
// fp16 PV, and the structure is CDNA4's:
//
//  * 4 waves x 32 query rows. S^T = K Q^T on v_mfma_f32_32x32x16_bf16 so a
//    lane owns one query row (lane % 32) and 32 of the 64 keys: the row max
//    and row sum are lane-local plus one xor-32 exchange.
//  * O^T = Vt P^T on the same MFMA, so P feeds the B operand straight from
//    the S^T accumulators and the rescale is lane-local. Vt comes from
//    vasc_pack_v with keys permuted into exactly the order the accumulators
//    hold them. The row sum is taken on the bf16-rounded P with v_dot2 so the
//    normaliser matches the P the MFMA consumes.
//  * Lazy rescaling: the running max only moves (and O is only rescaled)
//    when a block raises it by more than 8 in log2 units; P then stays below
//    2^8, far inside bf16 and fp32 range, and the result is unchanged up to
//    rounding. Most blocks skip the 32 multiplies.
//  * K and Vt tiles arrive through global_load_lds_dwordx4 straight into a
//    double-buffered LDS tile (2 x 16 KB), one block ahead of the MFMAs, with
//    a 16-byte-chunk xor swizzle ((row/2)%8) that spreads the 32 rows an
//    MFMA operand read touches over all LDS banks.
//  * Accumulators stay in VGPRs (built with -mllvm -amdgpu-mfma-vgpr-form,
//    no AGPR copies) and the kernel is held to 128 VGPRs so four waves share
//    each SIMD: one wave's MFMAs overlap another's exp/VALU work.
//  * workgroup ids are remapped so each XCD walks a contiguous range of
//    query blocks of the same head (K/V reuse in that XCD's L2).
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

constexpr float kLazyLog2 = 8.0f;  // rescale only when the max grows by > 2^8

template <bool kDense>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
void bsattn_fwd_kernel(const AttnParams p) {
  constexpr int CH = 512 / kThreads;  // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][2][kTile];

  const int64_t wg = xcd_remap(blockIdx.x, p.num_wg);
  const int qb = static_cast<int>(wg % p.nqb);
  const int64_t bh = wg / p.nqb;
  const int64_t h = bh % p.H;
  const int64_t b = bh / p.H;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, uniform
  const int l = tid & 63, lr = l & 31, hf = l >> 5;

  int n;
  const int32_t *list = nullptr;
  if (kDense) {
    n = static_cast<int>(p.nkb);
  } else {
    const int64_t row = bh * p.nqb + qb;
    list = p.idx + row * p.idx_w;
    n = p.cnt[row];
    n = n < 0 ? 0 : (n > p.idx_w ? static_cast<int>(p.idx_w) : n);
  }

  const int64_t qrow = static_cast<int64_t>(qb) * kBlockQ + w * 32 + lr;
  const bool qvalid = qrow < p.nq;
  uint16_t *optr = p.o + b * p.o_sb + h * p.o_sh + (qvalid ? qrow : 0) * p.o_st;

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
    const uint16_t *qptr = p.q + b * p.q_sb + h * p.q_sh + (qvalid ? qrow : 0) * p.q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qf[s] = qvalid ? *reinterpret_cast<const u32x4 *>(qptr + 16 * s + 8 * hf) : u32x4{0, 0, 0, 0};
  }

  // Staging: LDS chunk ci = u*256 + tid lands at byte 16*ci (global_load_lds
  // writes lane i of a wave at base + 16*i); it holds tile row ci/8, logical
  // chunk (ci%8) ^ swz(row), so each lane fetches that global chunk.
  const uint16_t *kbase = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t *vbase = p.vt + (bh * p.nkb) * kTile;
  const int nk32 = static_cast<int>(p.nk);
  const int nkb32 = static_cast<int>(p.nkb);
  int64_t koff[CH];
  int krow[CH], voff[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int ci = u * kThreads + tid;
    const int r = ci >> 3, c = (ci & 7) ^ swz(r);
    krow[u] = r;
    koff[u] = static_cast<int64_t>(r) * p.k_st + c * 8;
    voff[u] = r * kHeadDim + c * 8;
  }
  // Issue the loads of block blk into LDS buffer buf. Full blocks take the
  // precomputed per-thread offsets from a scalar block base; the partial last
  // block clamps its rows to the sequence end (their scores are masked).
  auto fetch = [&](int blk, int buf) {
    const int sb = (blk >= 0 && blk < nkb32) ? blk : 0;
    const uint16_t *kb = kbase + static_cast<int64_t>(sb) * kBlockK * p.k_st;
    const uint16_t *vb = vbase + static_cast<int64_t>(sb) * kTile;
    const bool full = (sb + 1) * kBlockK <= nk32;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const uint16_t *ks = kb + koff[u];
      if (!full) {
        const int t = sb * kBlockK + krow[u];
        if (t >= nk32) ks = kbase + static_cast<int64_t>(nk32 - 1) * p.k_st + (koff[u] - static_cast<int64_t>(krow[u]) * p.k_st);
      }
      uint16_t *kd = &smem[buf][0][(u * kThreads + w * 64) * 8];
      uint16_t *vd = &smem[buf][1][(u * kThreads + w * 64) * 8];
      __builtin_amdgcn_global_load_lds(ks, (__attribute__((address_space(3))) void *)kd, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vb + voff[u], (__attribute__((address_space(3))) void *)vd, 16, 0, 0);
    }
  };

  floatx16 oacc[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) { oacc[0][i] = 0.f; oacc[1][i] = 0.f; }
  float m = -INFINITY;  // running max in log2 units (stale by < kLazyLog2)
  float lsum = 0.f;

  // List entry j+1 is loaded during iteration j-1 (index clamped to the list)
  // so that reading it never waits on memory: the wait at the top of each
  // iteration already covers it.
  int blk = kDense ? 0 : __builtin_amdgcn_readfirstlane(list[0]);
  int32_t e_next = kDense ? 0 : list[n > 1 ? 1 : 0];
  fetch(blk, 0);
  for (int j = 0; j < n; ++j) {
    const int buf = j & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // block j landed; every wave is done with buffer buf^1
    const int cur = blk;
    if (j + 1 < n) {
      if (kDense) {
        blk = j + 1;
      } else {
        const int e = __builtin_amdgcn_readfirstlane(e_next);
        blk = p.delta ? blk + e : e;
        e_next = list[j + 2 < n ? j + 2 : n - 1];
      }
      fetch(blk, buf ^ 1);
    }
    const uint16_t *ks = smem[buf][0];
    const uint16_t *vs = smem[buf][1];

    // S^T tiles: keys 32t + [0,32) x this wave's 32 query rows.
    floatx16 sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[t][i] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 32 * t + lr;
        const u32x4 a = *reinterpret_cast<const u32x4 *>(ks + row * kHeadDim + ((2 * s + hf) ^ swz(row)) * 8);
        sacc[t] = mfma32(a, qf[s], sacc[t]);
      }

    // Mask keys past the sequence end and blocks outside [0, nkb).
    const bool blk_ok = cur >= 0 && cur < nkb32;
    const int lim = blk_ok ? nk32 - cur * kBlockK : 0;
    if (__builtin_expect(lim < kBlockK, 0)) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
          sacc[t][r] = kk < lim ? sacc[t][r] : -INFINITY;
        }
    }

    float mx = fmaxf(sacc[0][0], sacc[0][1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = fmaxf(mx, sacc[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[1][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx * p.c);
    const bool grow = m_new > m + kLazyLog2;
    if (__ballot(grow)) {
      const float alpha = grow ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) { oacc[0][r] *= alpha; oacc[1][r] *= alpha; }
      lsum *= alpha;
      m = grow ? m_new : m;
    }
    const float m_use = m == -INFINITY ? 0.f : m;

    // P^T as B operand: step s uses accumulators 8(s%2)..+7 of tile s/2.
    u32x4 pb[4];
    float ls = lsum;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int t = s >> 1, r = 8 * (s & 1);
      uint32_t d[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = __builtin_amdgcn_exp2f(fmaf(sacc[t][r + 2 * e], p.c, -m_use));
        const float x1 = __builtin_amdgcn_exp2f(fmaf(sacc[t][r + 2 * e + 1], p.c, -m_use));
        d[e] = pack_bf16x2(x0, x1);
        ls = add_bf16_pair(d[e], ls);
      }
      pb[s] = u32x4{d[0], d[1], d[2], d[3]};
    }
    lsum = ls;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        const int row = 32 * n2 + lr;
        const u32x4 a = *reinterpret_cast<const u32x4 *>(vs + row * kHeadDim + ((2 * s + hf) ^ swz(row)) * 8);
        oacc[n2] = mfma32(a, pb[s], oacc[n2]);
      }
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
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

int launch_attn(bool dense, const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st, const uint16_t *vt,
                uint16_t *o, int64_t o_sb, int64_t o_sh, int64_t o_st, int64_t B, int64_t H,
                int64_t nq, int64_t nk, int64_t d, const int32_t *idx, int64_t idx_w,
                const int32_t *cnt, int32_t delta, float sm_scale, void *stream) {
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
  VASC_REQUIRE(p.num_wg < (int64_t(1) << 31), "grid too large");
  VASC_SUPPORTED(nk < (int64_t(1) << 30) && nq < (int64_t(1) << 40), "sequence of %lld keys not built (< 2^30)",
                 (long long)nk);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dense)
    hipLaunchKernelGGL(bsattn_fwd_kernel<true>, dim3(p.num_wg), dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL(bsattn_fwd_kernel<false>, dim3(p.num_wg), dim3(kThreads), 0, s, p);
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

extern "C" int vasc_dense_attn_fwd(const uint16_t *q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                                   const uint16_t *k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                                   const uint16_t *vt, uint16_t *o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                                   int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t d, float sm_scale,
                                   void *stream) {
  return vasc::launch_attn(true, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, vt, o, o_sb, o_sh, o_st, B, H, nq,
                           nk, d, nullptr, 1, nullptr, 0, sm_scale, stream);
}
