// Device-side building blocks shared by every hxmi kernel (gfx950 / CDNA4 only).
//
// Vector types for MFMA operands, buffer-resource loads with hardware
// out-of-range zeroing, wave64 reductions, and the small math helpers the
// fused epilogues and row reductions use.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#define HXMI_LDS __attribute__((address_space(3)))

typedef _Float16 hx_half;
typedef __bf16 hx_bf16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int2v __attribute__((ext_vector_type(2)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_raw __attribute__((__vector_size__(8)));
typedef short i16x4_raw __attribute__((__vector_size__(8)));

namespace hxmi {

// Offset that is always beyond a buffer resource's num_records: a lane that
// loads from it receives zeros instead of touching memory.
constexpr uint32_t kOOB = 0x80000000u;

// Raw buffer resource for gfx9-family (CDNA) parts: base, no swizzle stride,
// num_records in bytes, dword3 = data-format word used for untyped loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16-byte global -> LDS copy that bypasses VGPRs. Lane i of the wave writes
// lds_wave_base + 16*i; voffset is this lane's byte offset into the buffer.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, HXMI_LDS void* lds_wave_base,
                                           uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_wave_base, 16, voffset, 0, 0, 0);
}

__device__ __forceinline__ int4v load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0);
}

// Same with the non-temporal cache policy (nt): for data read exactly once,
// e.g. decode weights; HBM streaming runs ~12 % faster on MI355X with it.
__device__ __forceinline__ int4v load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 2);
}

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// vmcnt(n) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ HXMI_LDS char* to_lds(char* p) { return (HXMI_LDS char*)(p); }

// Workgroup barrier over LDS filled by direct-to-LDS loads, after the
// caller's own partial wait for the loads it issued (wait_vmcnt<N>).
// __syncthreads() opens with a release fence on LDS, before which the
// compiler waits for every outstanding direct-to-LDS load (vmcnt(0)), the
// prefetched later stages included; this barrier keeps the caller's wait.
// It has the acquire half only (no LDS read moves above it), so it does not
// publish ds_write data or retire earlier LDS reads: use it where the only
// LDS data to share came in by direct loads and no stage is being refilled.
__device__ __forceinline__ void barrier_after_lds_loads() {
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Barrier of a pipelined K-step, after the caller's wait for the stage read
// next (wait_vmcnt<N>): every LDS read of this wave has returned
// (lgkmcnt(0)), so refill loads issued after it overwrite no stage that a
// wave still reads, and the later stages' loads stay in flight (they would
// not under __syncthreads(), as above).
__device__ __forceinline__ void barrier_before_refill() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt / expcnt untouched
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ds_read_b64_tr_b16: within each 16-lane group the 4x16 block of b16 values
// addressed by the lanes (lane L supplies row L/4, columns 4*(L%4)..+3) is
// returned transposed: lane i receives column i, rows 0..3.
// The pointer is __restrict__ so that the inlined read carries an alias
// scope: without one the compiler puts an s_waitcnt vmcnt(0) before every
// transposing read, draining each outstanding direct-to-LDS load (every
// prefetched K-step of a GEMM pipeline), which it does not do before plain
// LDS reads.  Callers order LDS reuse themselves, as for plain reads: a
// stage is read only after the wait and barrier that follow its loads.
__device__ __forceinline__ short4v lds_read_tr16(const char* __restrict__ p) {
  fp16x4_raw v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((HXMI_LDS fp16x4_raw*)(to_lds(const_cast<char*>(p))));
  return __builtin_bit_cast(short4v, v);
}

// Reductions over aligned groups of W lanes (16, 32 or the whole wave of 64)
// without LDS round trips: DPP swaps inside each row of 16 lanes (quad
// permutes, then rotations by 4 and 8 that cover the row), then
// v_permlane16_swap (pairs of rows: 32 lanes) and v_permlane32_swap (the
// two halves).  Every lane of a group receives its group's result.
template <int W = 64, typename Op>
__device__ __forceinline__ float wave_reduce_dpp(float v, Op op) {
  static_assert(W == 16 || W == 32 || W == 64, "group of 16, 32 or 64 lanes");
  auto dpp = [](float x, int ctrl) {
    switch (ctrl) {  // the control word must be a constant
      case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
      case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
      case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false));
      default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
    }
  };
  v = op(v, dpp(v, 0));  // quad_perm [1,0,3,2]
  v = op(v, dpp(v, 1));  // quad_perm [2,3,0,1]
  v = op(v, dpp(v, 2));  // row_ror:4
  v = op(v, dpp(v, 3));  // row_ror:8
  if (W == 16) return v;
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
  if (W == 32) return v;
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  return wave_reduce_dpp(v, [](float x, float y) { return fmaxf(x, y); });
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  return wave_reduce_dpp(v, [](float x, float y) { return x + y; });
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = width / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float fast_exp(float x) {
  // e^x = 2^(x*log2(e)); v_exp_f32 evaluates 2^x.
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// x * sigmoid(x).  The quotient is x times v_rcp_f32 of the denominator
// (within 1 ulp), not the IEEE division sequence (scale, fma chain, fixup),
// which cost several times as much in the GEMM epilogues; either is far
// inside the fp16 rounding of the result.  A denominator of +inf (x very
// negative) gives rcp 0 and the result -0, as the quotient does.
__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + fast_exp(-x)); }

// tanh-form GELU, 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715*x^3))), evaluated as
// x*sigmoid(2u) which equals it exactly in real arithmetic and avoids tanh's
// cancellation near 0 (the sigmoid's quotient as in silu).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  float u = k0 * (x + k1 * x * x * x);
  return x * __builtin_amdgcn_rcpf(1.0f + fast_exp(-2.0f * u));
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return (float)v;
}

template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return (T)v;
}

}  // namespace hxmi
