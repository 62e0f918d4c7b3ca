// GGUF block formats shared by every kernel: sizes, the IQ3_S codebook and its staging.
//
// The dequantised value of each format (computed in fp32, then rounded once to bf16 RNE):
// Q8_0 d*q; Q4_K (d*sc)*q - (dmin*m); Q6_K (d*sc)*(q-32); IQ3_S sign * ((d*(1+2*s))*g).
// Q8_0, IQ3_S and the Q4_K product are exact in fp32, so only the Q4_K subtraction and
// the Q6_K product round. The decoder is bpiece.h's BPiece<t> (the grouped GEMMs' operand
// decode, also run stand-alone by the dequant entry point).
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

// the codebook as byte selectors (one workgroup, call before a __syncthreads()): byte b of
// entry i is (m - 1) / 2 = m >> 1 for the magnitude m of the codebook's byte, the position
// 0..7 of m among the eight odd magnitudes 1..15 (the B-piece decoder's v_perm tables)
__device__ __forceinline__ void stage_iq3s_sel(uint32_t* lds_sel) {
  for (int i = threadIdx.x; i < 512; i += blockDim.x) lds_sel[i] = (c_iq3s_grid[i] >> 1) & 0x07070707u;
}

}  // namespace ktmi
