// Shared device/host helpers for the gfx950 kernels of librte_hip.
//
// Memory conventions used by every kernel in this library:
//   * bf16 tensors are passed as raw 16-bit words (uint16_t) holding the upper
//     half of an IEEE fp32; conversion fp32->bf16 is round-to-nearest-even.
//   * all index arrays are int32; all sizes that can exceed 2^31 elements are int64.
//   * kernels never allocate: callers pass outputs and workspaces.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace rte {

typedef uint16_t bf16;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_v;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_v;

__device__ __forceinline__ float bf2f(bf16 h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16, round to nearest even: the hardware conversion (v_cvt_pk_bf16_f32 on gfx950)
typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bf16 f2bf(float f) { return __builtin_bit_cast(bf16, (__bf16)f); }

// two fp32 -> one word of two bf16 (a in the low half), one conversion instruction
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  const f32x2_v v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Error reporting shared by all C-ABI entry points.
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// Small fill kernels (used instead of hipMemsetAsync so callers may capture graphs).
int fill_i32(int32_t* p, int32_t value, int64_t n, hipStream_t s);
int fill_f32(float* p, float value, int64_t n, hipStream_t s);

}  // namespace rte

#define RTE_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::rte::set_error(__VA_ARGS__);  \
      return -1;                      \
    }                                 \
  } while (0)

#define RTE_TRY(expr)          \
  do {                         \
    int _rc = (expr);          \
    if (_rc != 0) return _rc;  \
  } while (0)
