// Shared host/device helpers of the threadcut HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/threadcut_hip.h"

namespace tc {

// ---------------------------------------------------------------------------
// Host side: error state and device queries.
// ---------------------------------------------------------------------------

// Records a printf-style message for tc_last_error() on this thread and
// returns `code`, so validation reads `return fail(TC_ERR_..., "...")`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's message; called at the start of every entry point.
void clear_error();

// TC_OK if e == hipSuccess, else TC_ERR_HIP with the runtime's message.
int hip_status(hipError_t e, const char* what);

// Compute units of the current HIP device (cached per device id), or a
// negative TC_ERR_* code (negated) when no device is usable.
int current_device_cus(int* cus_out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device side: element conversions and wave64 data movement.
// ---------------------------------------------------------------------------

// One 32-bit word holds two 16-bit elements (little end first).
template <int DT> struct Elem;

template <> struct Elem<TC_DTYPE_F16> {
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ float lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
  // fp32 -> fp16, round to nearest even (v_cvt_f16_f32 in the default mode).
  static __device__ __forceinline__ uint32_t bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

template <> struct Elem<TC_DTYPE_BF16> {
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c, false);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // fp32 -> bf16, round to nearest even; NaN -> quiet NaN of the same sign.
  static __device__ __forceinline__ uint32_t bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  }
};

// DPP lane patterns inside each 16-lane row of a wave64 (GFX9 encodings).
enum : int {
  DPP_QUAD_XOR1 = 0xB1,      // quad_perm [1,0,3,2]
  DPP_QUAD_XOR2 = 0x4E,      // quad_perm [2,3,0,1]
  DPP_ROW_ROR4 = 0x124,      // row_ror:4
  DPP_ROW_ROR8 = 0x128,      // row_ror:8 (== lane ^ 8 in the row)
  DPP_ROW_HALF_MIRROR = 0x141,  // lane i <-> 7 - i in each half row
  DPP_ROW_NEWBCAST0 = 0x150  // + k: lane k of the row to the whole row
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Value of x held by lane k (0..15) of the caller's 16-lane row.
template <int K>
__device__ __forceinline__ float row_bcast(float x) {
  static_assert(K >= 0 && K < 16, "row lane");
  return dpp<DPP_ROW_NEWBCAST0 + K>(x);
}

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

}  // namespace tc
