// Kernel 5: token layout of the global-attention layer.
//
// The reference layer (attention.py:8351-8484, 8992-9030; tokens.py:2-126)
// splits the qkv projection into heads, applies q_norm / k_norm and the 2D
// rotary embedding, then makes six full copies to reach the [all patch
// tokens; all special tokens] order (reorder of q, k, v and extraction of
// the patch queries) and two more to return to frame-major order before the
// output projection. Here one pass reads each input element once and writes
// it once in its final place:
//
//   pack     q, k, v (frame-major: per frame S special tokens, then P-S
//            patch tokens) -> q_patch [B,H,Np,64], q_special [B,H,Ns,64],
//            k and v [B,H,T,64] in [patch; special] order, with optional
//            per-head LayerNorm of q and k and optional 2D rotary embedding,
//            in that order (fp32 arithmetic, one bf16 rounding per output);
//   restore  attention outputs in [patch; special] order -> frame-major
//            [B,T,H*64] (the layer's transpose + reshape before proj).
//
// Eight lanes own one (token, tensor, head) row of 64 features, 8 per lane,
// so a row is one 128-byte segment on both sides; the LayerNorm sums are
// xor butterflies inside the 8-lane group and the rotary partner of a
// feature (16 places away inside its half) sits two lanes away. A pack
// workgroup takes twelve groups of eight (token, tensor, head) rows in the
// order of the qkv projection, so its reads are one contiguous stretch and
// its 128-byte rows scatter on the write side; a wave's rows share token and
// tensor, which keeps the index arithmetic on the scalar unit (a restore
// workgroup takes 64 tokens of one head). A lane issues all of its loads
// before it uses the first.
// Precedent in the reference: kernels/qkv_layout.py:8-157 (layout only).
#include "innovation.h"

namespace vasc {
namespace {

constexpr int kHeadDim = 64;
constexpr int kThreads = 256;
constexpr int kRows = kThreads / 8;  // token rows per pass: 8 lanes per 64-feature row
// rows per lane group: three for the pack kernel (64 VGPRs or fewer, eight
// waves per SIMD), two for the copy-only restore
constexpr int kPackPasses = 3;
constexpr int kPackGroups = 4 * kPackPasses;  // row groups of eight per pack workgroup
constexpr int kPasses = 2;
constexpr int kTokens = kRows * kPasses;

struct PackParams {
  const uint16_t *src[3];       // q, k, v: element (b, t, h, d) at src + b*sb + t*st + h*sh + d
  int64_t sb[3], st[3], sh[3];
  int32_t H, N, P, S;           // T = N * P frame-major tokens
  const void *norm_w[2], *norm_b[2];
  float eps[2];
  int32_t norm[2];              // LayerNorm of q (0) and k (1): 0 none, 1 fp32 parameters, 2 bf16 parameters
  const int32_t *pos;           // (row, column) position of token (b, t) at pos + b*pos_sb + t*pos_st
  int64_t pos_sb, pos_st;
  const float *rope_cos, *rope_sin;  // [rope_n, 16]: cos/sin of position p times frequency i
  int32_t rope_n;
  uint16_t *q_patch, *q_special, *k_out, *v_out;
  // pack_global_kernel only: V as MFMA tiles, the pooled means and the pair innovation
  uint16_t *vt, *pooled_q, *pooled_k, *pooled_v;
  float *innovation;
};


// LayerNorm weight and bias of q (0) and k (1) into LDS, 1 and 0 where
// absent (one thread per staged value; the caller synchronises before use).
__device__ __forceinline__ void stage_norms(const PackParams &p, floatx4 (&nrm)[2][2][kHeadDim / 4], int tid) {
  static_assert(kThreads == 2 * 2 * kHeadDim, "one thread per staged LayerNorm weight or bias");
  if (!(p.norm[0] || p.norm[1])) return;
  const int which = tid >> 7, wb = (tid >> 6) & 1, f = tid & 63;
  // a tensor without the norm may pass any pointer: read only the normed one's
  const void *src = !p.norm[which] ? nullptr : (wb == 0 ? p.norm_w[which] : p.norm_b[which]);
  float val = wb == 0 ? 1.f : 0.f;
  if (src)
    val = p.norm[which] == 2 ? bf16_to_f32(static_cast<const uint16_t *>(src)[f]) : static_cast<const float *>(src)[f];
  reinterpret_cast<float *>(nrm[which][wb])[f] = val;
}

// One (token, tensor, head) row, this lane's 8 features 8 sub .. 8 sub + 7 of
// raw bf16 input: per-head LayerNorm (q, k with their norm on) and the 2D
// rotary embedding at position pq (q, k when positions are given), in
// float32. part: 0 q, 1 k, 2 v (v passes through).
__device__ __forceinline__ void transform_row(const PackParams &p, const floatx4 (&nrm)[2][2][kHeadDim / 4],
                                              const u32x4 &raw, int part, int32_t pq, int sub, float (&x)[8]) {
  const bool norm = part < 2 && p.norm[part == 0 ? 0 : 1];
  const bool rope = part < 2 && p.pos;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = bf16_to_f32(static_cast<uint16_t>(raw[e]));
    x[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(raw[e] >> 16));
  }
  if (norm) {
    const int pn = part == 0 ? 0 : 1;
    const floatx4 w0 = nrm[pn][0][2 * sub], w1 = nrm[pn][0][2 * sub + 1];
    const floatx4 b0 = nrm[pn][1][2 * sub], b1 = nrm[pn][1][2 * sub + 1];
    const float eps = part == 0 ? p.eps[0] : p.eps[1];
    // statistics in float32 with fused multiply-adds and the hardware
    // reciprocal square root (about one ulp): the output is rounded to bf16
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += x[e];
    const float mean = group8_sum(s) * (1.0f / kHeadDim);
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] -= mean;
      v = fmaf(x[e], x[e], v);
    }
    const float var = group8_sum(v) * (1.0f / kHeadDim);
    const float rstd = __builtin_amdgcn_rsqf(var + eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float we = e < 4 ? w0[e] : w1[e - 4], be = e < 4 ? b0[e] : b1[e - 4];
      x[e] = fmaf(x[e] * rstd, we, be);
    }
  }
  if (rope) {
    // features [0, 32) rotate with the row position, [32, 64) with the
    // column position; inside a half, feature j < 16 pairs with j + 16
    const int32_t q = pq < 0 ? 0 : (pq >= p.rope_n ? p.rope_n - 1 : pq);
    const floatx4 *c4 = reinterpret_cast<const floatx4 *>(p.rope_cos + q * 16 + (sub & 1) * 8);
    const floatx4 *s4 = reinterpret_cast<const floatx4 *>(p.rope_sin + q * 16 + (sub & 1) * 8);
    const floatx4 c0 = c4[0], c1 = c4[1], s0 = s4[0], s1 = s4[1];
    const bool first = (sub & 2) == 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float partner = dpp<kQuadXor2>(x[e]);
      const float rot = first ? -partner : partner;
      const float ce = e < 4 ? c0[e] : c1[e - 4], se = e < 4 ? s0[e] : s1[e - 4];
      x[e] = fmaf(rot, se, x[e] * ce);
    }
  }
}


// Workgroup (x, b): row groups [12 x, +12) of batch entry b. A row group is
// eight (token, tensor, head) rows of one token and one tensor: group g is
// token g / G, tensor (g % G) / H8 (0 q, 1 k, 2 v) and heads 8 ((g % G) % H8)
// onward, with H8 = ceil(H / 8) groups per tensor and G = 3 H8 (2 H8 when v is
// not packed). Wave w takes groups 4i + w of the range in passes i = 0..2, so
// the token and the tensor of every row a wave holds are wave-uniform (the
// address arithmetic is scalar); lane group j of the wave takes head 8 (..) + j
// (lanes past H idle). For the usual [B, T, 3, H, 64] qkv projection a
// workgroup reads one contiguous stretch of it; the 128-byte rows scatter on
// the write side. The LayerNorm weights are staged in LDS once per
// workgroup; the rotary table entries of a row are loaded when the row is
// computed.
__global__ __launch_bounds__(kThreads) void pack_qkv_kernel(const PackParams p) {
  const int32_t H = p.H, T = p.N * p.P;
  const int32_t H8 = (H + 7) >> 3, G = (p.v_out ? 3 : 2) * H8;
  const int32_t groups = T * G;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, sub = tid & 7, hl = (tid >> 3) & 7;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __shared__ floatx4 nrm[2][2][kHeadDim / 4];
  const bool any_norm = p.norm[0] || p.norm[1];
  stage_norms(p, nrm, tid);
  bool ok[kPackPasses];
  int32_t tk[kPackPasses], pt[kPackPasses], hd[kPackPasses];
  u32x4 raw[kPackPasses];
  int32_t pq[kPackPasses];
#pragma unroll
  for (int i = 0; i < kPackPasses; ++i) {
    const int32_t grp = static_cast<int32_t>(blockIdx.x) * (4 * kPackPasses) + 4 * i + w;
    const bool gv = grp < groups;
    const int32_t g = gv ? grp : groups - 1;  // in-bounds stand-in for groups past the end
    const int32_t t = __builtin_amdgcn_readfirstlane(g / G);
    const int32_t rem = g - t * G;
    const int32_t part = __builtin_amdgcn_readfirstlane(rem / H8);
    const int32_t h = (rem - part * H8) * 8 + hl;
    ok[i] = gv && h < H;
    const int32_t hc = h < H ? h : H - 1;
    tk[i] = t; pt[i] = part; hd[i] = hc;
    const uint16_t *base = part == 0 ? p.src[0] : (part == 1 ? p.src[1] : p.src[2]);
    const int64_t sb = part == 0 ? p.sb[0] : (part == 1 ? p.sb[1] : p.sb[2]);
    const int64_t st = part == 0 ? p.st[0] : (part == 1 ? p.st[1] : p.st[2]);
    const int64_t sh = part == 0 ? p.sh[0] : (part == 1 ? p.sh[1] : p.sh[2]);
    raw[i] = *reinterpret_cast<const u32x4 *>(base + b * sb + static_cast<int64_t>(t) * st + hc * sh + sub * 8);
    pq[i] = p.pos ? p.pos[b * p.pos_sb + static_cast<int64_t>(t) * p.pos_st + (sub >> 2)] : 0;
  }
  const int32_t np = p.N * (p.P - p.S), ns = p.N * p.S;
  if (any_norm) __syncthreads();
#pragma unroll
  for (int i = 0; i < kPackPasses; ++i) {
    const int part = pt[i];
    float x[8];
    transform_row(p, nrm, raw[i], part, pq[i], sub, x);
    if (!ok[i]) continue;
    u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
    const int32_t n = tk[i] / p.P, tf = tk[i] - n * p.P;
    const bool patch = tf >= p.S;
    const int32_t ip = n * (p.P - p.S) + (tf - p.S), is = n * p.S + tf;
    const int64_t bh = b * H + hd[i];
    uint16_t *dst;
    if (part == 0)
      dst = patch ? p.q_patch + (bh * np + ip) * kHeadDim : p.q_special + (bh * ns + is) * kHeadDim;
    else
      dst = (part == 1 ? p.k_out : p.v_out) + (bh * T + (patch ? ip : np + is)) * kHeadDim;
    *reinterpret_cast<u32x4 *>(dst + sub * 8) = out;
  }
}

// The global layer's layout pass with the pooling and the V tiles fused in.
// Workgroup (x, b): head x % H and positions [128 (x / H), +128) of the
// [patch; special] order of batch entry b, i.e. query block x / H and key
// blocks 2 (x / H) and 2 (x / H) + 1. Each thread holds, for four positions
// 32 u + (tid >> 3), the 16-byte feature chunk tid & 7 of q, k and v; q and
// k take transform_row (bit-identical to pack_qkv_kernel) and are written
// as there; v goes through LDS into its two [64 d][64 key] MFMA tiles (the
// layout and key permutation of pack_v_kernel, zero past the end). From the
// bf16-rounded q, k and v of the patch positions the workgroup sums, in
// float32 (per thread over its positions, across the 8 row groups of a wave,
// then the four waves in order), the means of its query block and of its
// two key blocks (as pool_qkv_kernel: the tail blocks average their real
// tokens), rounds them to bf16 and computes the pair innovation of its two
// V blocks (an odd tail pairs with itself). Replaces pack_qkv_kernel,
// pool_qkv_kernel and pack_v_kernel in a global layer: the packed q, k
// and V tiles are read back by nothing but the attention.
__global__ __launch_bounds__(kThreads) void pack_global_kernel(const PackParams p) {
  constexpr int kTilePad = 8;  // LDS row padding of the V tiles
  __shared__ floatx4 nrm[2][2][kHeadDim / 4];
  __shared__ uint16_t tile[2][kHeadDim][kHeadDim + kTilePad];  // [key block][d][key]
  __shared__ float red[4][5][kHeadDim];                        // per wave: q, k0, k1, v0, v1 sums
  __shared__ float pvm[2][kHeadDim];                           // the two pooled V rows (bf16 values)
  const int32_t H = p.H, T = p.N * p.P;
  const int32_t np = p.N * (p.P - p.S), ns = p.N * p.S;
  const int32_t h = static_cast<int32_t>(blockIdx.x % H);
  const int32_t blk = static_cast<int32_t>(blockIdx.x / H);
  const int64_t b = blockIdx.y;
  const int64_t bh = b * H + h;
  const int tid = threadIdx.x, sub = tid & 7, r = tid >> 3, w = tid >> 6, lane = tid & 63;
  stage_norms(p, nrm, tid);

  u32x4 raw[3][4];
  int32_t pq[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int32_t i = blk * 128 + 32 * u + r;  // position in [patch; special] order
    const bool in = i < T;
    int32_t t = 0;
    if (in) {
      if (i < np) {
        const int32_t n = i / (p.P - p.S);
        t = n * p.P + p.S + (i - n * (p.P - p.S));
      } else {
        const int32_t is = i - np, n = is / p.S;
        t = n * p.P + (is - n * p.S);
      }
    }
#pragma unroll
    for (int X = 0; X < 3; ++X)
      raw[X][u] = in ? *reinterpret_cast<const u32x4 *>(p.src[X] + b * p.sb[X] + static_cast<int64_t>(t) * p.st[X] +
                                                         h * p.sh[X] + sub * 8)
                     : u32x4{0, 0, 0, 0};
    pq[u] = p.pos && in ? p.pos[b * p.pos_sb + static_cast<int64_t>(t) * p.pos_st + (sub >> 2)] : 0;
  }
  if (p.norm[0] || p.norm[1]) __syncthreads();

  float acc[5][8];  // q, k (block 0, 1), v (block 0, 1) sums of this thread's patch positions
#pragma unroll
  for (int j = 0; j < 5; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int32_t i = blk * 128 + 32 * u + r;
    const bool in = i < T, patch = i < np;
    const int half = u >> 1;
#pragma unroll
    for (int X = 0; X < 2; ++X) {
      float x[8];
      transform_row(p, nrm, raw[X][u], X, pq[u], sub, x);
      u32x4 out;
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
      if (in) {
        uint16_t *dst = X == 0 ? (patch ? p.q_patch + (bh * np + i) * kHeadDim
                                        : p.q_special + (bh * ns + (i - np)) * kHeadDim)
                               : p.k_out + (bh * T + i) * kHeadDim;
        *reinterpret_cast<u32x4 *>(dst + sub * 8) = out;
      }
      if (patch) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[X == 0 ? 0 : 1 + half][2 * e] += __uint_as_float(out[e] << 16);
          acc[X == 0 ? 0 : 1 + half][2 * e + 1] += __uint_as_float(out[e] & 0xffff0000u);
        }
      }
    }
    // v: bf16 as read (zero past the end) into its tile, and its sums
    const int key = 32 * (u & 1) + r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[half][sub * 8 + 2 * e][key] = static_cast<uint16_t>(raw[2][u][e]);
      tile[half][sub * 8 + 2 * e + 1][key] = static_cast<uint16_t>(raw[2][u][e] >> 16);
      if (patch) {
        acc[3 + half][2 * e] += __uint_as_float(raw[2][u][e] << 16);
        acc[3 + half][2 * e + 1] += __uint_as_float(raw[2][u][e] & 0xffff0000u);
      }
    }
  }
  // Sums of the 40 partials (flat index 8 j + e) across the 8 row groups of
  // the wave (lane bits 3-5), reduced and scattered at once: a 32-lane
  // permlane swap of partials i and i + 20 leaves the lower lanes summing
  // i and the upper lanes i + 20, a 16-lane swap of i and i + 10 splits
  // again, and a DPP row rotate by 8 finishes. Lane bits 5 and 4 then name
  // the ten partials a lane holds (flat index t + 10 b4 + 20 b5).
  float g[20], hs[10];
#pragma unroll
  for (int i = 0; i < 20; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[i >> 3][i & 7]),
                                                    __float_as_uint(acc[(i + 20) >> 3][(i + 20) & 7]), false, false);
    g[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(g[i]), __float_as_uint(g[i + 10]), false, false);
    hs[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    hs[i] += xor_lane(hs[i], 8);
  }
  if ((lane & 8) == 0) {
    const int first = 10 * ((lane >> 4) & 1) + 20 * (lane >> 5);
#pragma unroll
    for (int t = 0; t < 10; ++t) {
      const int i = first + t;
      red[w][i >> 3][sub * 8 + (i & 7)] = hs[t];
    }
  }
  __syncthreads();

  // the two V tiles, keys permuted to the attention kernel's operand order
  const int32_t nkb = (T + 63) / 64;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int32_t j = 2 * blk + half;
    if (j >= nkb) break;
    uint16_t *dst = p.vt + (bh * nkb + j) * (64 * kHeadDim);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ci = tid + 256 * u;
      const int d = ci >> 3, chunk = ci & 7;
      const int s4 = chunk >> 1, hh = chunk & 1;
      uint16_t o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = tile[half][d][16 * s4 + 8 * (e >> 2) + 4 * hh + (e & 3)];
      *reinterpret_cast<u32x4 *>(dst + d * 64 + chunk * 8) = *reinterpret_cast<const u32x4 *>(o);
    }
  }

  // pooled means: q over the query block, k and v over each key block
  const int32_t qb = (np + 127) / 128, kb = (np + 63) / 64;
  for (int item = tid; item < 5 * kHeadDim; item += kThreads) {
    const int d = item & 63, j = item >> 6;
    const float sum = (red[0][j][d] + red[1][j][d]) + (red[2][j][d] + red[3][j][d]);
    int32_t count;
    uint16_t *dst;
    if (j == 0) {
      count = np - blk * 128;
      count = count > 128 ? 128 : count;
      dst = p.pooled_q ? p.pooled_q + (bh * qb + blk) * kHeadDim : nullptr;
    } else {
      const int half = (j - 1) & 1;
      const int32_t kblk = 2 * blk + half;
      count = np - kblk * 64;
      count = count > 64 ? 64 : count;
      uint16_t *base = j <= 2 ? p.pooled_k : p.pooled_v;
      dst = base ? base + (bh * kb + kblk) * kHeadDim : nullptr;
    }
    if (count <= 0) continue;
    const uint16_t mean = f32_to_bf16(sum / static_cast<float>(count));
    if (dst) dst[d] = mean;
    if (j >= 3) pvm[j - 3][d] = bf16_to_f32(mean);
  }
  if (!p.innovation) return;
  __syncthreads();
  if (w == 0 && 2 * blk < kb) {
    const float lv = pvm[0][lane];
    const float rv = 2 * blk + 1 < kb ? pvm[1][lane] : lv;
    const float iota = pair_innovation_wave(lv, rv);
    if (lane == 0) p.innovation[bh * ((kb + 1) / 2) + blk] = iota;
  }
}

struct RestoreParams {
  const uint16_t *xp, *xs;      // [B,H,Np,64] and [B,H,Ns,64], element (b,h,i,d) at x + b*sb + h*sh + i*st + d
  int64_t p_sb, p_sh, p_st, s_sb, s_sh, s_st;
  int32_t H, N, P, S;
  uint16_t *out;                // [B, T, H*64] contiguous
};

// Workgroup (x, b): head x % H, tokens [64 (x / H), +64) of batch entry b;
// consecutive workgroups fill the heads of the same output tokens.
__global__ __launch_bounds__(kThreads) void restore_tokens_kernel(const RestoreParams p) {
  const int32_t H = p.H, T = p.N * p.P;
  const int32_t h = static_cast<int32_t>(blockIdx.x % H);
  const int32_t tb = static_cast<int32_t>(blockIdx.x / H);
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, sub = tid & 7;
  u32x4 v[kPasses];
#pragma unroll
  for (int i = 0; i < kPasses; ++i) {
    const int32_t t = tb * kTokens + i * kRows + (tid >> 3);
    if (t < T) {
      const int32_t n = t / p.P, tf = t - n * p.P;
      const uint16_t *src = tf >= p.S
          ? p.xp + b * p.p_sb + h * p.p_sh + static_cast<int64_t>(n * (p.P - p.S) + tf - p.S) * p.p_st
          : p.xs + b * p.s_sb + h * p.s_sh + static_cast<int64_t>(n * p.S + tf) * p.s_st;
      v[i] = *reinterpret_cast<const u32x4 *>(src + sub * 8);
    }
  }
#pragma unroll
  for (int i = 0; i < kPasses; ++i) {
    const int32_t t = tb * kTokens + i * kRows + (tid >> 3);
    if (t < T) *reinterpret_cast<u32x4 *>(p.out + ((b * T + t) * H + h) * kHeadDim + sub * 8) = v[i];
  }
}

int check_src(const char *name, const void *ptr, int64_t sb, int64_t st, int64_t sh) {
  VASC_REQUIRE(ptr != nullptr, "%s is NULL", name);
  VASC_REQUIRE((reinterpret_cast<uintptr_t>(ptr) & 15) == 0, "%s must be 16-byte aligned", name);
  VASC_REQUIRE(sb >= 0 && st >= 0 && sh >= 0 && sb % 8 == 0 && st % 8 == 0 && sh % 8 == 0,
               "%s strides (%lld,%lld,%lld) must be non-negative multiples of 8 elements", name, (long long)sb,
               (long long)st, (long long)sh);
  return VASC_OK;
}

}  // namespace
}  // namespace vasc

extern "C" int vasc_pack_qkv(const uint16_t *q, int64_t q_sb, int64_t q_st, int64_t q_sh, const uint16_t *k,
                             int64_t k_sb, int64_t k_st, int64_t k_sh, const uint16_t *v, int64_t v_sb,
                             int64_t v_st, int64_t v_sh, int64_t B, int64_t H, int64_t N, int64_t P, int64_t S,
                             int64_t d, const void *q_norm_w, const void *q_norm_b, float q_eps,
                             int32_t q_norm, const void *k_norm_w, const void *k_norm_b, float k_eps,
                             int32_t k_norm, const int32_t *pos, int64_t pos_sb, int64_t pos_st,
                             const float *rope_cos, const float *rope_sin, int64_t rope_n, uint16_t *q_patch,
                             uint16_t *q_special, uint16_t *k_out, uint16_t *v_out, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == kHeadDim, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(B > 0 && H > 0 && N > 0 && P > 0 && S >= 0 && S <= P, "invalid sizes B=%lld H=%lld N=%lld P=%lld S=%lld",
               (long long)B, (long long)H, (long long)N, (long long)P, (long long)S);
  VASC_REQUIRE(B < 65536 && H < 4096 && N * P < (int64_t(1) << 31) / 64, "too many tokens or heads");
  VASC_REQUIRE(N * P * 3 * ((H + 7) / 8) < (int64_t(1) << 31) - kPackGroups, "too many (token, head) rows");
  int rc;
  if ((rc = check_src("q", q, q_sb, q_st, q_sh))) return rc;
  if ((rc = check_src("k", k, k_sb, k_st, k_sh))) return rc;
  if (v_out && (rc = check_src("v", v, v_sb, v_st, v_sh))) return rc;
  VASC_REQUIRE(k_out, "k_out is required");
  VASC_REQUIRE(P == S || q_patch, "q_patch is required when frames hold patch tokens");
  VASC_REQUIRE(S == 0 || q_special, "q_special is required when frames hold special tokens");
  for (const void *o : {static_cast<const void *>(q_patch), static_cast<const void *>(q_special),
                        static_cast<const void *>(k_out), static_cast<const void *>(v_out)})
    VASC_REQUIRE((reinterpret_cast<uintptr_t>(o) & 15) == 0, "outputs must be 16-byte aligned");
  VASC_REQUIRE(q_norm >= 0 && q_norm <= 2 && k_norm >= 0 && k_norm <= 2,
               "q_norm / k_norm must be 0 (none), 1 (fp32 parameters) or 2 (bf16 parameters)");
  VASC_REQUIRE(q_norm == 0 || q_eps >= 0.f, "q_eps must be non-negative");
  VASC_REQUIRE(k_norm == 0 || k_eps >= 0.f, "k_eps must be non-negative");
  if (pos) {
    VASC_REQUIRE(rope_cos && rope_sin && rope_n > 0, "rotary tables are required with positions");
    VASC_REQUIRE(((reinterpret_cast<uintptr_t>(rope_cos) | reinterpret_cast<uintptr_t>(rope_sin)) & 15) == 0,
                 "rotary tables must be 16-byte aligned");
    VASC_REQUIRE(pos_sb >= 0 && pos_st >= 2, "position strides must be pos_sb >= 0, pos_st >= 2");
  }
  PackParams p;
  p.src[0] = q; p.src[1] = k; p.src[2] = v;
  p.sb[0] = q_sb; p.st[0] = q_st; p.sh[0] = q_sh;
  p.sb[1] = k_sb; p.st[1] = k_st; p.sh[1] = k_sh;
  p.sb[2] = v_sb; p.st[2] = v_st; p.sh[2] = v_sh;
  p.H = static_cast<int32_t>(H); p.N = static_cast<int32_t>(N); p.P = static_cast<int32_t>(P);
  p.S = static_cast<int32_t>(S);
  p.norm_w[0] = q_norm_w; p.norm_b[0] = q_norm_b; p.eps[0] = q_eps; p.norm[0] = q_norm;
  p.norm_w[1] = k_norm_w; p.norm_b[1] = k_norm_b; p.eps[1] = k_eps; p.norm[1] = k_norm;
  p.pos = pos; p.pos_sb = pos_sb; p.pos_st = pos_st;
  p.rope_cos = rope_cos; p.rope_sin = rope_sin;
  p.rope_n = static_cast<int32_t>(rope_n < (int64_t(1) << 30) ? rope_n : (int64_t(1) << 30));
  p.q_patch = q_patch; p.q_special = q_special; p.k_out = k_out; p.v_out = v_out;
  hipLaunchKernelGGL(pack_qkv_kernel, dim3(static_cast<unsigned>(cdiv(N * P * (v_out ? 3 : 2) * ((H + 7) / 8), kPackGroups)), static_cast<unsigned>(B)),
                     dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), p);
  return check_launch("vasc_pack_qkv");
}

extern "C" int vasc_pack_global(const uint16_t *q, int64_t q_sb, int64_t q_st, int64_t q_sh, const uint16_t *k,
                                int64_t k_sb, int64_t k_st, int64_t k_sh, const uint16_t *v, int64_t v_sb,
                                int64_t v_st, int64_t v_sh, int64_t B, int64_t H, int64_t N, int64_t P, int64_t S,
                                int64_t d, const void *q_norm_w, const void *q_norm_b, float q_eps, int32_t q_norm,
                                const void *k_norm_w, const void *k_norm_b, float k_eps, int32_t k_norm,
                                const int32_t *pos, int64_t pos_sb, int64_t pos_st, const float *rope_cos,
                                const float *rope_sin, int64_t rope_n, uint16_t *q_patch, uint16_t *q_special,
                                uint16_t *k_out, uint16_t *vt, uint16_t *pooled_q, uint16_t *pooled_k,
                                uint16_t *pooled_v, float *innovation, void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == kHeadDim, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(B > 0 && H > 0 && N > 0 && P > 0 && S >= 0 && S < P, "invalid sizes B=%lld H=%lld N=%lld P=%lld S=%lld",
               (long long)B, (long long)H, (long long)N, (long long)P, (long long)S);
  VASC_REQUIRE(B < 65536 && H < 4096 && N * P < (int64_t(1) << 31) / 64, "too many tokens or heads");
  VASC_REQUIRE(cdiv(N * P, 128) * H < (int64_t(1) << 31), "grid too large");
  int rc;
  if ((rc = check_src("q", q, q_sb, q_st, q_sh))) return rc;
  if ((rc = check_src("k", k, k_sb, k_st, k_sh))) return rc;
  if ((rc = check_src("v", v, v_sb, v_st, v_sh))) return rc;
  VASC_REQUIRE(q_patch && k_out && vt, "q_patch, k_out and vt are required");
  VASC_REQUIRE(S == 0 || q_special, "q_special is required when frames hold special tokens");
  for (const void *o : {static_cast<const void *>(q_patch), static_cast<const void *>(q_special),
                        static_cast<const void *>(k_out), static_cast<const void *>(vt)})
    VASC_REQUIRE((reinterpret_cast<uintptr_t>(o) & 15) == 0, "outputs must be 16-byte aligned");
  VASC_REQUIRE(q_norm >= 0 && q_norm <= 2 && k_norm >= 0 && k_norm <= 2,
               "q_norm / k_norm must be 0 (none), 1 (fp32 parameters) or 2 (bf16 parameters)");
  VASC_REQUIRE(q_norm == 0 || q_eps >= 0.f, "q_eps must be non-negative");
  VASC_REQUIRE(k_norm == 0 || k_eps >= 0.f, "k_eps must be non-negative");
  if (pos) {
    VASC_REQUIRE(rope_cos && rope_sin && rope_n > 0, "rotary tables are required with positions");
    VASC_REQUIRE(((reinterpret_cast<uintptr_t>(rope_cos) | reinterpret_cast<uintptr_t>(rope_sin)) & 15) == 0,
                 "rotary tables must be 16-byte aligned");
    VASC_REQUIRE(pos_sb >= 0 && pos_st >= 2, "position strides must be pos_sb >= 0, pos_st >= 2");
  }
  PackParams p{};
  p.src[0] = q; p.src[1] = k; p.src[2] = v;
  p.sb[0] = q_sb; p.st[0] = q_st; p.sh[0] = q_sh;
  p.sb[1] = k_sb; p.st[1] = k_st; p.sh[1] = k_sh;
  p.sb[2] = v_sb; p.st[2] = v_st; p.sh[2] = v_sh;
  p.H = static_cast<int32_t>(H); p.N = static_cast<int32_t>(N); p.P = static_cast<int32_t>(P);
  p.S = static_cast<int32_t>(S);
  p.norm_w[0] = q_norm_w; p.norm_b[0] = q_norm_b; p.eps[0] = q_eps; p.norm[0] = q_norm;
  p.norm_w[1] = k_norm_w; p.norm_b[1] = k_norm_b; p.eps[1] = k_eps; p.norm[1] = k_norm;
  p.pos = pos; p.pos_sb = pos_sb; p.pos_st = pos_st;
  p.rope_cos = rope_cos; p.rope_sin = rope_sin;
  p.rope_n = static_cast<int32_t>(rope_n < (int64_t(1) << 30) ? rope_n : (int64_t(1) << 30));
  p.q_patch = q_patch; p.q_special = q_special; p.k_out = k_out; p.v_out = nullptr;
  p.vt = vt; p.pooled_q = pooled_q; p.pooled_k = pooled_k; p.pooled_v = pooled_v; p.innovation = innovation;
  hipLaunchKernelGGL(pack_global_kernel, dim3(static_cast<unsigned>(cdiv(N * P, 128) * H), static_cast<unsigned>(B)),
                     dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), p);
  return check_launch("vasc_pack_global");
}

extern "C" int vasc_restore_tokens(const uint16_t *x_patch, int64_t p_sb, int64_t p_sh, int64_t p_st,
                                   const uint16_t *x_special, int64_t s_sb, int64_t s_sh, int64_t s_st, int64_t B,
                                   int64_t H, int64_t N, int64_t P, int64_t S, int64_t d, uint16_t *out,
                                   void *stream) {
  using namespace vasc;
  VASC_SUPPORTED(d == kHeadDim, "head_dim %lld not built (built: 64)", (long long)d);
  VASC_REQUIRE(B > 0 && H > 0 && N > 0 && P > 0 && S >= 0 && S <= P, "invalid sizes");
  VASC_REQUIRE(B < 65536 && H < 4096 && N * P < (int64_t(1) << 31) / 64, "too many tokens or heads");
  VASC_REQUIRE(cdiv(N * P, kTokens) * 3 * H < (int64_t(1) << 31), "grid too large");
  VASC_REQUIRE(out && (reinterpret_cast<uintptr_t>(out) & 15) == 0, "out must be a 16-byte aligned buffer");
  int rc;
  if (P > S && (rc = check_src("x_patch", x_patch, p_sb, p_st, p_sh))) return rc;
  if (S > 0 && (rc = check_src("x_special", x_special, s_sb, s_st, s_sh))) return rc;
  RestoreParams p;
  p.xp = x_patch; p.p_sb = p_sb; p.p_sh = p_sh; p.p_st = p_st;
  p.xs = x_special; p.s_sb = s_sb; p.s_sh = s_sh; p.s_st = s_st;
  p.H = static_cast<int32_t>(H); p.N = static_cast<int32_t>(N); p.P = static_cast<int32_t>(P);
  p.S = static_cast<int32_t>(S);
  p.out = out;
  hipLaunchKernelGGL(restore_tokens_kernel, dim3(static_cast<unsigned>(cdiv(N * P, kTokens) * H), static_cast<unsigned>(B)),
                     dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), p);
  return check_launch("vasc_restore_tokens");
}
