// GGUF super-block decoders: 16 consecutive values of a weight row to fp32.
//
// Every function returns the exact fp32 value of the format's dequantisation with a
// fixed operation order and no fused multiply-add: Q8_0 d*q; Q4_K (d*sc)*q - (dmin*m);
// Q6_K (d*sc)*q; IQ3_S sign * ((d*(1+2*s))*g). Q8_0, IQ3_S and the Q4_K product are
// exact in fp32, so only the Q4_K subtraction and the Q6_K second product round.
// Rounding the result to bf16 (RNE) gives the dequantised bf16 weights.
//
// Byte layouts (little endian), per block:
//   Q8_0  (32 values, 34 B): fp16 d @0, int8 qs[32] @2
//   Q4_K  (256 values, 144 B): fp16 d @0, fp16 dmin @2, u8 scales[12] @4, u8 qs[128] @16
//   Q6_K  (256 values, 210 B): u8 ql[128] @0, u8 qh[64] @128, int8 scales[16] @192, fp16 d @208
//   IQ3_S (256 values, 110 B): fp16 d @0, u8 qs[64] @2, u8 qh[8] @66, u8 signs[32] @74,
//                              u8 scales[4] @106
// Reference: hot/kt_gguf_moe_multi/ggml-common.h:55-61, 88-94, 105-112, 145-154;
// value formulas hot/kt_gguf_moe_multi/vecdotq.cuh:1326-1367 (Q4_K scale/min unpack),
// :1625-1648 (Q6_K), :1875-1899 and P:11397-11420 (IQ3_S).
#pragma once
#include "ktmi_common.h"

namespace ktmi {

// Q4_K 6-bit scale and min of sub-block j (0..7) from the 12 scale bytes.
__device__ __forceinline__ void q4k_scale_min(const uint8_t* scales, int j, int& sc, int& m) {
  if (j < 4) {
    sc = scales[j] & 63;
    m = scales[j + 4] & 63;
  } else {
    sc = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4);
    m = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
  }
}

// ---- 16 values starting at element e0 (a multiple of 16) of a row whose bytes start at
// `row`. The row must be at least 2-byte aligned (Q4_K: 16-byte aligned).

__device__ __forceinline__ void decode16_q8_0(const uint8_t* row, int e0, float y[16]) {
  const uint8_t* b = row + (e0 / QK8_0) * QB8_0;
  const float d = half_bits_to_float(ld_u16(b));
  uint32_t w[4];
  ld16_a2(b + 2 + (e0 % QK8_0), w);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = (int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xFF);
    y[i] = d * (float)q;
  }
}

__device__ __forceinline__ void decode16_q4_k(const uint8_t* row, int e0, float y[16]) {
  const uint8_t* b = row + (e0 / QK_K) * QB4_K;
  const int o = e0 % QK_K;
  const int g = o / 64, l0 = o % 64;
  const int j = 2 * g + (l0 >= 32);
  const uint32_t dm = *(const uint32_t*)b;
  const float d = half_bits_to_float(dm & 0xFFFF);
  const float dmin = half_bits_to_float(dm >> 16);
  int sc, m;
  q4k_scale_min(b + 4, j, sc, m);
  const float d1 = d * (float)sc;
  const float m1 = dmin * (float)m;
  uint32_t w[4];
  ld16_a16(b + 16 + 32 * g + (l0 % 32), w);
  const int shift = (l0 >= 32) ? 4 : 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int q = (w[i >> 2] >> (8 * (i & 3) + shift)) & 0xF;
    y[i] = __fsub_rn(__fmul_rn(d1, (float)q), m1);
  }
}

__device__ __forceinline__ void decode16_q6_k(const uint8_t* row, int e0, float y[16]) {
  const uint8_t* b = row + (e0 / QK_K) * QB6_K;
  const int o = e0 % QK_K;
  const int h = o / 128, r = o % 128;
  const int c = r / 32, l0 = r % 32;
  const float d = half_bits_to_float(ld_u16(b + 208));
  const int sc = (int8_t)b[192 + 8 * h + l0 / 16 + 2 * c];
  const float d1 = d * (float)sc;
  uint32_t lo[4], hi[4];
  ld16_a2(b + 64 * h + l0 + 32 * (c & 1), lo);
  ld16_a2(b + 128 + 32 * h + l0, hi);
  const int lshift = (c < 2) ? 0 : 4;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int nib = (lo[i >> 2] >> (8 * (i & 3) + lshift)) & 0xF;
    const int hb = (hi[i >> 2] >> (8 * (i & 3) + 2 * c)) & 3;
    const int q = (nib | (hb << 4)) - 32;
    y[i] = __fmul_rn(d1, (float)q);
  }
}

// grid: the 512-entry IQ3_S codebook (LDS or global)
__device__ __forceinline__ void decode16_iq3_s(const uint8_t* row, int e0, const uint32_t* grid, float y[16]) {
  const uint8_t* b = row + (e0 / QK_K) * QBIQ3_S;
  const int o = e0 % QK_K;
  const int ib = o / 32, lbase = (o % 32) / 8;  // lbase in {0, 2}
  const float d = half_bits_to_float(ld_u16(b));
  const int nib = (b[106 + ib / 2] >> (4 * (ib % 2))) & 15;
  const float db = d * (float)(1 + 2 * nib);
  const int qh = b[66 + ib];
#pragma unroll
  for (int li = 0; li < 2; ++li) {
    const int l = lbase + li;
    const int sg = b[74 + 4 * ib + l];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int idx = b[2 + 8 * ib + 2 * l + sub] | (((qh >> (2 * l + sub)) & 1) << 8);
      const uint32_t gv = grid[idx];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int jj = 4 * sub + k;
        const float v = __fmul_rn(db, (float)((gv >> (8 * k)) & 0xFF));
        y[8 * li + jj] = ((sg >> jj) & 1) ? -v : v;
      }
    }
  }
}

template <int TYPE>
__device__ __forceinline__ void decode16(const uint8_t* row, int e0, const uint32_t* grid, float y[16]) {
  if constexpr (TYPE == GGML_Q8_0) {
    decode16_q8_0(row, e0, y);
  } else if constexpr (TYPE == GGML_Q4_K) {
    decode16_q4_k(row, e0, y);
  } else if constexpr (TYPE == GGML_Q6_K) {
    decode16_q6_k(row, e0, y);
  } else {
    decode16_iq3_s(row, e0, grid, y);
  }
}

template <int TYPE>
struct Fmt;
template <>
struct Fmt<GGML_Q8_0> { static constexpr int QK = QK8_0, QB = QB8_0; };
template <>
struct Fmt<GGML_Q4_K> { static constexpr int QK = QK_K, QB = QB4_K; };
template <>
struct Fmt<GGML_Q6_K> { static constexpr int QK = QK_K, QB = QB6_K; };
template <>
struct Fmt<GGML_IQ3_S> { static constexpr int QK = QK_K, QB = QBIQ3_S; };

static __constant__ uint32_t c_iq3s_grid[512] = {
#include "iq3s_grid.inc"
};

// copy the codebook into LDS (one workgroup), call before a __syncthreads()
__device__ __forceinline__ void stage_iq3s_grid(uint32_t* lds_grid) {
  for (int i = threadIdx.x; i < 512; i += blockDim.x) lds_grid[i] = c_iq3s_grid[i];
}

}  // namespace ktmi
