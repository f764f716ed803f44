// Shared helpers for the gfx950 kernels of libvoom_hip.so: vector types, bf16
// conversion, wave reductions, error reporting and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/voom_hip.h"

namespace voom {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950), as bits.
__device__ __forceinline__ uint16_t f2bf(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

__device__ __forceinline__ float bf2f(uint16_t x) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(x) << 16);
}

// Packs two fp32 values into one dword of two bf16 (low half = a).
// One v_cvt_pk_bf16_f32 (round to nearest even, as f2bf).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// a.lo + a.hi (+ c) of two packed bf16 values in fp32: one v_dot2_f32_bf16
// against (1, 1).
__device__ __forceinline__ float sum_bf16x2(uint32_t a, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), one, c, false);
}

__device__ __forceinline__ float wave_max_across_groups(float v) {
  // Reduces over lanes l, l^16, l^32, l^48 (the four 16-lane groups).
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum_across_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Sum over the 64 lanes, the same value in every lane, in a fixed order:
// xor 1 and xor 2 within each quad, then the mirrored half of each 8-lane
// group, then the mirrored half of each 16-lane row (all DPP moves, after
// which every lane of a row holds the row's sum), then rows 0 + 16 + 32 + 48
// read out left to right.  Cheaper than a shuffle butterfly, whose six steps
// each round-trip through the LDS crossbar.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_uniform(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return ((r0 + r1) + r2) + r3;
}

// Maximum over the 64 lanes, the same value in every lane (the moves of
// wave_sum_uniform with fmaxf).
__device__ __forceinline__ float wave_max_uniform(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Inclusive prefix sum over the 64 lanes (lane l gets x_0 + ... + x_l), all
// by DPP: shifts right by 1, 2, 4 and 8 within each 16-lane row (a lane with
// no source adds 0), then lane 15 of rows 0 and 2 added into rows 1 and 3,
// and lane 31 into rows 2 and 3.  A shuffle ladder would take six round
// trips through the LDS crossbar instead.
__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
  (void)lane;
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
  return x;
}

// Marks a wave-uniform value as such (v_readfirstlane_b32 into an SGPR).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Waits until every vector-memory load of this wave has landed (vmcnt(0);
// expcnt and lgkmcnt untouched).  Emitted through the s_waitcnt builtin so
// the compiler's wait-count pass sees it: after an inline-asm wait that pass
// still counts older loads (say, operands loaded before a loop) as pending
// and inserts waits of its own before their uses, which then also wait for
// every load issued since.
__device__ __forceinline__ void wait_vmem_all() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// operations, then s_barrier.  Unlike __syncthreads() it does not drain
// outstanding global loads, so register prefetches and direct-to-LDS loads
// stay in flight across it.  The wait and the barrier are builtins, which the
// compiler's wait-count pass sees; the empty asm statements only stop the
// compiler from moving memory accesses across the barrier.  (With the wait
// and barrier written as inline asm, the pass no longer told the LDS buffers
// apart after the barrier and put a vmcnt(0) before LDS accesses that no
// pending direct-to-LDS load writes -- in the MLA kernel before the P reads,
// i.e. a wait for the whole next tile.)
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // gfx9 encoding: lgkmcnt 0, vmcnt 63, expcnt 7
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Hardware base-2 exponential (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- host side -------------------------------------------------------------

// Records a printf-style message for voom_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
// Converts a HIP status into the ABI return convention (0 or positive code).
int check_hip(hipError_t e, const char* what);
// Number of compute units of the current device (cached per device).
int device_cu_count();

inline bool is_pow2(long long x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(long long x) {
  int s = 0;
  while ((1LL << s) < x) ++s;
  return s;
}

}  // namespace voom

#define VOOM_REQUIRE(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::voom::set_error(VOOM_EINVAL, __VA_ARGS__); \
  } while (0)

#define VOOM_LAUNCH_CHECK(what) ::voom::check_hip(hipGetLastError(), what)
