// Shared device/host helpers of the gfx950 sparse global-attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/vasc_hip.h"

namespace vasc {

// ---------------------------------------------------------------- host side
// Thread-local error string behind vasc_last_error() (defined in capi.cpp).
void set_error(const char *fmt, ...);

#define VASC_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::vasc::set_error(__VA_ARGS__);    \
      return VASC_ERR_ARGUMENT;          \
    }                                    \
  } while (0)

#define VASC_SUPPORTED(cond, ...)        \
  do {                                   \
    if (!(cond)) {                       \
      ::vasc::set_error(__VA_ARGS__);    \
      return VASC_ERR_UNSUPPORTED;       \
    }                                    \
  } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char *what);

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// ---------------------------------------------------------------- device side
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even float -> bfloat16 bits (NaN -> canonical quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(f32_to_bf16(f));
}

// Two floats -> packed bf16x2 with the hardware RNE conversion.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  floatx2 f = {a, b};
  bf16x2 h = __builtin_convertvector(f, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// Cross-lane moves inside groups of 8 lanes by DPP: xor 1 and xor 2 are
// quad permutations, and the half-row mirror (lane i <-> 7 - i) reaches the
// other quad of the group.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xb1;   // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4e;   // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141;

__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, dpp<kQuadXor1>(v));
  v = fmaxf(v, dpp<kQuadXor2>(v));
  return fmaxf(v, dpp<kHalfMirror>(v));
}

__device__ __forceinline__ float group8_sum(float v) {
  v += dpp<kQuadXor1>(v);
  v += dpp<kQuadXor2>(v);
  return v + dpp<kHalfMirror>(v);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  return (uint64_t(1) << lane_id()) - 1;
}

// Number of set bits of a wave mask below this lane (v_mbcnt_lo/hi).
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

// The value of lane (lane ^ off) for off in {1, 2, 4, 8, 16, 32}, by VALU
// cross-lane moves instead of an LDS permute: DPP quad permutations (1, 2),
// row shifts selected by lane bit 2 (4), a row rotate by 8 (8), and gfx950's
// v_permlane16_swap / v_permlane32_swap, which exchange rows of 16 / 32
// lanes (16, 32). `off` must be a constant after unrolling.
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int off) {
  const int lane = __lane_id();
  switch (off) {
    case 1: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xb1, 0xf, 0xf, false));
    case 2: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4e, 0xf, 0xf, false));
    case 4: {
      const uint32_t up = __builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x104, 0xf, 0xf, false);  // row_shl:4
      const uint32_t dn = __builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x114, 0xf, 0xf, false);  // row_shr:4
      return (lane & 4) ? dn : up;
    }
    case 8: return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x128, 0xf, 0xf, false));
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
  }
}
__device__ __forceinline__ int xor_lane(int v, int off) {
  return static_cast<int>(xor_lane(static_cast<uint32_t>(v), off));
}
__device__ __forceinline__ float xor_lane(float v, int off) {
  return __uint_as_float(xor_lane(__float_as_uint(v), off));
}
__device__ __forceinline__ double xor_lane(double v, int off) {
  const uint64_t u = __double_as_longlong(v);
  const uint64_t lo = xor_lane(static_cast<uint32_t>(u), off), hi = xor_lane(static_cast<uint32_t>(u >> 32), off);
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// Canonical 64-lane xor butterfly of float64 lane sums (offsets 32..1).
__device__ __forceinline__ double wave_butterfly(double s) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s = s + xor_lane(s, off);
  return s;
}

// Integer and max reductions keep the LDS permute: the kernels that use them
// are VALU-bound, and one ds_bpermute per stage costs them less than the
// VALU moves.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// LDS DMA: global memory straight into LDS without a register round trip.
// Lane i of the wave writes its chunk at lds_addr + size*i. Issued through
// asm (M0, which holds the LDS address, is saved and restored) so the
// compiler does not see an LDS write it would drain with s_waitcnt vmcnt(0)
// before every later LDS read: callers pace the DMA with their own vmcnt
// waits, and a lane whose exec bit is clear loads nothing.
__device__ __forceinline__ void lds_dma16(const void *sbase, uint32_t voff_bytes, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(voff_bytes), "s"(sbase)
      : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *sbase, uint32_t voff_bytes, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dword %2, %3\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(voff_bytes), "s"(sbase)
      : "memory");
}
// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr32(const void *ptr) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)ptr));
}

// Maps the hardware workgroup id to a logical id so that each of the 8 XCDs
// (which receive workgroups round-robin) processes one contiguous range of
// logical ids, keeping neighbouring tiles of one head in one L2.
__device__ __forceinline__ int64_t xcd_remap(int64_t pid, int64_t num) {
  constexpr int64_t kXcd = 8;
  const int64_t q = num / kXcd, r = num % kXcd;
  const int64_t xcd = pid % kXcd, local = pid / kXcd;
  return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

}  // namespace vasc
