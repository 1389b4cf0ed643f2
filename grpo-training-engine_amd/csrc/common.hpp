// Shared device helpers and C-ABI error plumbing for libgrpo_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/grpo_hip.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

namespace grpo {

// ---------------------------------------------------------------- errors --
void set_error(const char* fmt, ...);

inline int einval(const char* what) {
  set_error("invalid argument: %s", what);
  return GRPO_EINVAL;
}

inline int hip_check(hipError_t e, const char* where) {
  if (e == hipSuccess) return GRPO_OK;
  set_error("%s: %s", where, hipGetErrorString(e));
  return (int)e > 0 ? (int)e : 1;
}

// Launch status of the kernel just enqueued (catches bad launch configs).
inline int launch_check(const char* name) { return hip_check(hipGetLastError(), name); }

inline hipStream_t as_stream(grpo_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Lets kernel KERN use up to BYTES of dynamic LDS, less its static LDS (the
// two share gfx950's 160 KiB): hipFuncSetAttribute once per kernel (the kernel
// is a template argument because the instantiations of one kernel template
// share a function type).
template <auto KERN, int BYTES>
int allow_dynamic_lds() {
  static const int rc = [] {
    hipFuncAttributes fa{};
    if (int e = hip_check(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(KERN)),
                          "hipFuncGetAttributes"))
      return e;
    return hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(KERN),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         BYTES - (int)fa.sharedSizeBytes),
                     "hipFuncSetAttribute");
  }();
  return rc;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

__host__ __device__ inline bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}
__host__ __device__ inline bool aligned8(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 7u) == 0;
}

// ---------------------------------------------------------------- bf16 ---
// float -> bf16 round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
// Round a float to the nearest bf16 value, returned as float.
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
// Two floats -> packed bf16 pair (lo in bits 0..15): one v_cvt_pk_bf16_f32.
typedef float float2_v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const float2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// float16 (IEEE half) counterparts, round-to-nearest-even.  The empty asm
// keeps f a float32 value: without it the compiler contracts a product feeding
// the conversion into v_fma_mixlo_f16 (one rounding of the exact product, and
// -0 * ... + 0 = +0), where the reference rounds the float32 product first.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float round_h(float f) { return h2f(f2h(f)); }
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}
// The 16-bit float type of a kernel instance: bf16 (F16 = false) or float16.
template <bool F16>
__device__ __forceinline__ uint16_t f2e(float f) { return F16 ? f2h(f) : f2bf(f); }
template <bool F16>
__device__ __forceinline__ float e2f(uint16_t b) { return F16 ? h2f(b) : bf2f(b); }
template <bool F16>
__device__ __forceinline__ float round_e(float f) { return F16 ? round_h(f) : round_bf(f); }
template <bool F16>
__device__ __forceinline__ uint32_t pack_e2(float lo, float hi) {
  return F16 ? pack_h2(lo, hi) : pack_bf2(lo, hi);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Reductions over the lane pairs {l, l^16} and {l, l^32} of a wave with
// v_permlane16_swap / v_permlane32_swap (VALU; no LDS crossbar).  The swap
// leaves the lower lane's value in r[0] and the upper lane's in r[1] in both
// lanes of a pair, so both get the same (lower op upper) result.
__device__ __forceinline__ float pair16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Kernel arguments are read with scalar loads that the compiler places where a
// field is first needed; a kernel whose early branches use fields from several
// 64-byte lines of the argument segment then waits for one scalar-cache miss
// after another (each a memory round trip at kernel start).  Touching every
// line of the first BYTES bytes at entry issues those misses together; the
// later argument loads hit the scalar cache.
template <int BYTES>
__device__ __forceinline__ void touch_kernargs() {
  constexpr int LINES = (BYTES + 63) / 64;
  static_assert(LINES <= 8, "argument segment larger than 512 bytes");
  typedef const __attribute__((address_space(4))) uint32_t* kernarg_ptr;
  const kernarg_ptr k = (kernarg_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t v[8];
#pragma unroll
  for (int i = 0; i < LINES; ++i) v[i] = k[i * 16];
#pragma unroll
  for (int i = 0; i < LINES; ++i) asm volatile("" ::"s"(v[i]));
}

// Value from a wave-uniform address that no thread writes during the kernel,
// read through the constant address space: a scalar load, whose wait
// (lgkmcnt) does not hold back the wave's vector loads.  (A plain load of a
// uniform address is a vector load that must be waited for, and moved to a
// scalar register, before the loads that follow it can be issued.)
template <typename T>
__device__ __forceinline__ T load_uniform(const T* ptr) {
  typedef const __attribute__((address_space(4))) T* cptr;
  return *(cptr)ptr;
}

// 16-byte load of data read once per step (NF4 weights, K/V blocks) with the
// non-temporal hint, so the stream does not evict what other workgroups
// re-read from L2 (staged x, partial sums, absmax lines).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum over the 64 lanes of a wave, every lane gets the total: DPP within each
// row of 16 lanes (quad_perm xor 1, xor 2, half-row mirror, row mirror), then
// the permlane swaps across rows.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over each aligned group of 8 lanes (every lane of the group gets it):
// DPP quad_perm xor 1, xor 2, then the half-row mirror (lane i + lane 7 - i).
__device__ __forceinline__ float sum8(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  return v;
}
// The same over each DPP row of 16 lanes (then the row mirror, lane i + 15 - i).
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return pair32_sum(pair16_sum(v));
}

// Eight columns of the RMSNorm output bf16(bf16(h * inv) * w) (the reference's
// rounding points, as add_rmsnorm_kernel), h and w in natural order.
__device__ __forceinline__ uint4 norm8(uint4 hv, uint4 wv, float inv) {
  const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = pack_bf2(round_bf(bf_lo(hw[q]) * inv) * bf_lo(ww[q]),
                    round_bf(bf_hi(hw[q]) * inv) * bf_hi(ww[q]));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// ------------------------------------------------ same-XCD hand-over ------
// Several kernels hand a group's partial results to the last-arriving
// workgroup of the group through an L2 atomic counter and plain stores.  That
// is correct only if every workgroup of the group runs on one XCD (one L2):
// the launches give a group's workgroups equal linear ids modulo 8, and the
// dispatcher places workgroup i on XCD (i + c) mod 8 (c fixed per launch).
// The assumption is checked, not trusted: every arrival adds 1 to a 4-bit
// field of the counter selected by the XCD it runs on (HW_REG_XCC_ID), so
//  * a group on one XCD ends with n arrivals in one field (the last arriver
//    resets the counter to zero);
//  * a group whose arrivals reach one counter from two XCDs ends with two
//    non-zero fields: the arriver that completes the count sets *err;
//  * a group split over two L2s never completes a count in either: its
//    counter is left non-zero.
// The host reads the counters and *err after a run; non-zero means the
// hand-over was not on one XCD and the results of that run are not valid.

// XCD of the calling wave (hardware register 20 = XCC_ID, bits 3:0).
__device__ __forceinline__ uint32_t xcc_id() {
  return (uint32_t)__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;
}

// Sum of the eight 4-bit fields of v.
__device__ __forceinline__ uint32_t nibble_sum(uint32_t v) {
  v = (v & 0x0F0F0F0Fu) + ((v >> 4) & 0x0F0F0F0Fu);
  v += v >> 8;
  v += v >> 16;
  return v & 0xFFu;
}

// One arrival of a group of n <= 15 workgroups at *cnt (called by one thread,
// after the workgroup's stores are acknowledged).  Returns true for the
// arrival that completes the group; that one resets *cnt.
__device__ __forceinline__ bool xcd_arrive(int* cnt, int n, int* err) {
  const uint32_t x = xcc_id();
  const uint32_t inc = 1u << (4 * (x & 7u));
  const uint32_t old = (uint32_t)__hip_atomic_fetch_add(cnt, (int)inc, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_WORKGROUP);
  const uint32_t now = old + inc;
  if (nibble_sum(now) != (uint32_t)n) return false;
  if (x > 7u || now != (uint32_t)n << (4 * (x & 7u))) {
    if (err) *err = 1;
  }
  *cnt = 0;
  return true;
}

__device__ __forceinline__ f32x4_t mfma16x16x32(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
// v_mfma_f32_16x16x32_f16 (F16) or _bf16 on operands given as 16-bit patterns.
template <bool F16>
__device__ __forceinline__ f32x4_t mfma16x16x32_e(uint4 a, uint4 b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return mfma16x16x32(a, b, c);
}

}  // namespace grpo
