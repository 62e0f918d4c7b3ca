// Shared definitions for the ktmi HIP library (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ktmi.h"

// ggml type ids (the GGUF tensor type field)
#define GGML_Q8_0 8
#define GGML_Q4_K 12
#define GGML_Q6_K 14
#define GGML_IQ3_S 21

// super-block geometry: (values per block, bytes per block)
#define QK8_0 32
#define QB8_0 34
#define QK_K 256
#define QB4_K 144
#define QB6_K 210
#define QBIQ3_S 110
#define QK8_1 32
#define QB8_1 36

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
// the same vectors with 4-byte alignment (36-byte q8_1 blocks, 2-byte aligned GGUF blocks
// read from the dword below them)
typedef uint32_t u32x4_a4_t __attribute__((ext_vector_type(4))) __attribute__((aligned(4)));
typedef uint32_t u32x2_a4_t __attribute__((ext_vector_type(2))) __attribute__((aligned(4)));

namespace ktmi {

// set by host entry points; returned by ktmi_last_error()
void set_error(const char* fmt, ...);
void clear_error();

#define KTMI_HIP_TRY(expr)                                                               \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess) {                                                              \
      ::ktmi::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                        __LINE__);                                                       \
      return KTMI_EHIP;                                                                  \
    }                                                                                    \
  } while (0)

#define KTMI_REQUIRE(cond, code, ...) \
  do {                                \
    if (!(cond)) {                    \
      ::ktmi::set_error(__VA_ARGS__); \
      return (code);                  \
    }                                 \
  } while (0)

__host__ __device__ inline int64_t blck_size(int t) {
  switch (t) {
    case GGML_Q8_0: return QK8_0;
    case GGML_Q4_K: case GGML_Q6_K: case GGML_IQ3_S: return QK_K;
    default: return 0;
  }
}
__host__ __device__ inline int64_t type_size(int t) {
  switch (t) {
    case GGML_Q8_0: return QB8_0;
    case GGML_Q4_K: return QB4_K;
    case GGML_Q6_K: return QB6_K;
    case GGML_IQ3_S: return QBIQ3_S;
    default: return 0;
  }
}
__host__ __device__ inline int64_t row_bytes(int64_t cols, int t) { return cols / blck_size(t) * type_size(t); }
__host__ __device__ inline int64_t q8_1_cols_padded(int64_t cols) { return (cols + 511) / 512 * 512; }
__host__ __device__ inline int64_t q8_1_row_bytes(int64_t cols) { return q8_1_cols_padded(cols) / 32 * QB8_1; }

// ---------------------------------------------------------------- device helpers

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// fp32 -> bf16 with round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Loads through explicitly global pointers: a weight address read from a slot table is a
// generic pointer to the compiler, which would otherwise emit flat loads (those also wait
// on the LDS counter).
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

// little-endian loads from 2-byte aligned addresses (GGUF blocks of 34/110/210 bytes
// are only 2-byte aligned)
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) { return gload<uint16_t>(p); }
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
  return (uint32_t)gload<uint16_t>(p) | ((uint32_t)gload<uint16_t>(p + 2) << 16);
}
// 16 bytes from a 2-byte aligned address as 4 little-endian dwords
__device__ __forceinline__ void ld16_a2(const uint8_t* p, uint32_t w[4]) {
  uint16_t h[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = gload<uint16_t>(p + 2 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
}
__device__ __forceinline__ void ld16_a16(const uint8_t* p, uint32_t w[4]) {
  u32x4_t v = gload<u32x4_t>(p);
  w[0] = v[0];
  w[1] = v[1];
  w[2] = v[2];
  w[3] = v[3];
}

}  // namespace ktmi
