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
//    the S^T accumulators and the rescale by exp2(m_old - m_new) is
//    lane-local. Vt comes from vasc_pack_v with keys permuted into exactly
//    the order the accumulators hold them.
//  * K and Vt tiles are double-buffered in LDS (2 x 16 KB) with an xor
//    swizzle of the 16-byte chunks (chunk ^ row%8) so every ds_read_b128 of
//    an MFMA operand is bank-conflict free; the next block's global loads
//    are in flight during the current block's MFMAs.
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

template <bool kDense>
__global__ __launch_bounds__(kThreads) void bsattn_fwd_kernel(const AttnParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[2][2][kTile];

  const int64_t wg = xcd_remap(blockIdx.x, p.num_wg);
  const int qb = static_cast<int>(wg % p.nqb);
  const int64_t bh = wg / p.nqb;
  const int64_t h = bh % p.H;
  const int64_t b = bh / p.H;
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, lr = l & 31, hf = l >> 5;

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

  // Global -> LDS staging: thread owns LDS chunks tid and tid + 256, i.e.
  // rows r0 = tid/8 and r0 + 32 at physical chunk tid%8, which holds logical
  // chunk (tid%8) ^ (row%8) (identical for both rows).
  const int r0 = tid >> 3;
  const int lchunk = (tid & 7) ^ (r0 & 7);
  const uint16_t *kbase = p.k + b * p.k_sb + h * p.k_sh + lchunk * 8;
  const uint16_t *vbase = p.vt + (bh * p.nkb) * kTile + lchunk * 8;

  auto block_at = [&](int j, int64_t prev) -> int64_t {
    if (kDense) return j;
    const int32_t e = list[j];
    return p.delta ? prev + e : static_cast<int64_t>(e);
  };
  auto fetch = [&](int64_t blk, u32x4 &k0, u32x4 &k1, u32x4 &v0, u32x4 &v1) {
    const bool ok = blk >= 0 && blk < p.nkb;
    const int64_t sb = ok ? blk : 0;
    int64_t t0 = sb * kBlockK + r0, t1 = t0 + 32;
    t0 = t0 < p.nk ? t0 : p.nk - 1;
    t1 = t1 < p.nk ? t1 : p.nk - 1;
    k0 = *reinterpret_cast<const u32x4 *>(kbase + t0 * p.k_st);
    k1 = *reinterpret_cast<const u32x4 *>(kbase + t1 * p.k_st);
    const uint16_t *vb = vbase + sb * kTile;
    v0 = *reinterpret_cast<const u32x4 *>(vb + r0 * kHeadDim);
    v1 = *reinterpret_cast<const u32x4 *>(vb + (r0 + 32) * kHeadDim);
  };

  floatx16 oacc[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) { oacc[0][i] = 0.f; oacc[1][i] = 0.f; }
  float m = -INFINITY;
  float lsum = 0.f;

  int64_t blk = block_at(0, 0);
  u32x4 pk0, pk1, pv0, pv1;
  fetch(blk, pk0, pk1, pv0, pv1);

  for (int j = 0; j < n; ++j) {
    const int buf = j & 1;
    uint16_t *ks = smem[buf][0];
    uint16_t *vs = smem[buf][1];
    *reinterpret_cast<u32x4 *>(ks + tid * 8) = pk0;
    *reinterpret_cast<u32x4 *>(ks + (tid + 256) * 8) = pk1;
    *reinterpret_cast<u32x4 *>(vs + tid * 8) = pv0;
    *reinterpret_cast<u32x4 *>(vs + (tid + 256) * 8) = pv1;
    __syncthreads();

    const int64_t cur = blk;
    if (j + 1 < n) {
      blk = block_at(j + 1, blk);
      fetch(blk, pk0, pk1, pv0, pv1);
    }

    // S^T tiles: keys 32t + [0,32) x this wave's 32 query rows.
    floatx16 sacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[t][i] = 0.f;
      const int row = 32 * t + lr;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int chunk = (2 * s + hf) ^ (row & 7);
        const u32x4 a = *reinterpret_cast<const u32x4 *>(ks + row * kHeadDim + chunk * 8);
        sacc[t] = mfma32(a, qf[s], sacc[t]);
      }
    }

    // Mask keys past the sequence end and blocks outside [0, nkb).
    const bool blk_ok = cur >= 0 && cur < p.nkb;
    if (!blk_ok || (cur + 1) * kBlockK > p.nk) {
      const int64_t base = cur * kBlockK;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * t + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (!blk_ok || base + kk >= p.nk) sacc[t][r] = -INFINITY;
        }
    }

    float mx = sacc[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[1][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx * p.c);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    m = m_new;

    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = __builtin_amdgcn_exp2f(fmaf(sacc[t][r], p.c, -m_use));
        sacc[t][r] = e;
        psum += e;
      }
    lsum = lsum * alpha + psum;
#pragma unroll
    for (int r = 0; r < 16; ++r) { oacc[0][r] *= alpha; oacc[1][r] *= alpha; }

    // P^T as B operand: step s uses accumulators 8(s%2)..+7 of tile s/2.
    u32x4 pb[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int t = s >> 1, r = 8 * (s & 1);
      pb[s] = u32x4{pack_bf16x2(sacc[t][r + 0], sacc[t][r + 1]), pack_bf16x2(sacc[t][r + 2], sacc[t][r + 3]),
                    pack_bf16x2(sacc[t][r + 4], sacc[t][r + 5]), pack_bf16x2(sacc[t][r + 6], sacc[t][r + 7])};
    }
#pragma unroll
    for (int n2 = 0; n2 < 2; ++n2) {
      const int row = 32 * n2 + lr;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int chunk = (2 * s + hf) ^ (row & 7);
        const u32x4 a = *reinterpret_cast<const u32x4 *>(vs + row * kHeadDim + chunk * 8);
        oacc[n2] = mfma32(a, pb[s], oacc[n2]);
      }
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
