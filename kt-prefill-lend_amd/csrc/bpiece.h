// B-tile pieces for the grouped MFMA GEMMs: one thread's 32 dequantised weights of one
// row for one 64-value K step, as 16 packed bf16 words.
//
// Each format is split into load() (global loads only, into registers) and decode()
// (ALU only), so a kernel can issue the loads of step k+1 before the MFMAs of step k and
// decode after them. The values are the exact dequantisation of formats.h rounded once
// to bf16 (Q4_K uses an FMA: d*sc*q is exact in fp32, so fma(d*sc, q, -dmin*m) rounds the
// same value as the separate multiply and subtract).
//
// K steps: a 256-value super-block column sb is 4 steps SUB = 0..3 of 64 values (SUB is a
// template parameter: every field position is then a compile-time constant). 256 sb +
// ksub<SUB>() + coff(q) is the row offset of the step's 8-value chunk q (q = 0..7, step
// positions 8q..8q+7); the activation tile uses the same map, so any permutation of K
// inside a super-block is fine for the product. Natural order (ksub = 64 SUB, coff = 8 q)
// except Q6_K, whose step SUB = 2 h + c covers the two 32-runs of half h that share their
// ql/qh bytes: 128 h + 32 c + [0, 32) and the same + 64.
// Piece h (0 or 1) of a step covers:
//   Q4_K : positions [16h, 16h+16) and [32+16h, +16): the two nibbles of qs bytes
//          [32g+16h, +16), g = SUB (sub-blocks 2g and 2g+1)
//   Q6_K : positions [16h, +16) (run c, low nibbles of ql and bits 2c of qh) and
//          [32+16h, +16) (run c+2, high nibbles and bits 2c+4 of the same bytes)
//   Q8_0, IQ3_S: positions [32h, 32h+32) (one Q8_0 block, one IQ3_S 32-group)
// `off0`/`off1` give the step positions of out[0..7] and out[8..15] (16 values each).
//
// 2-byte aligned blocks (Q8_0 34 B, Q6_K 210 B, IQ3_S 110 B) are read with dword loads
// from the dword-aligned address below and realigned with v_alignbyte; every dword read
// holds at least one byte of the block, so no load leaves the tensor's pages.
#pragma once
#include "formats.h"

namespace ktmi {

__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t shift) {
  return __builtin_amdgcn_alignbyte(hi, lo, shift);
}
__device__ __forceinline__ const uint32_t* dword_floor(const uint8_t* p) {
  return (const uint32_t*)((uintptr_t)p & ~(uintptr_t)3);
}
__device__ __forceinline__ uint32_t byte_shift(const uint8_t* p) { return (uint32_t)((uintptr_t)p & 3); }

template <int TYPE>
struct BPiece;

template <>
struct BPiece<GGML_Q4_K> {
  struct Raw { u32x4_t hdr, q; };
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  __device__ static int coff(int q) { return 8 * q; }
  template <int SUB>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + sb * QB4_K;
    r.hdr = gload<u32x4_t>(b);
    r.q = gload<u32x4_t>(b + 16 + 32 * SUB + 16 * h);
  }
  template <int SUB>
  __device__ static void decode(const Raw& r, const uint32_t*, uint32_t out[16]) {
    const float d = half_bits_to_float(r.hdr[0] & 0xFFFF);
    const float dmin = half_bits_to_float(r.hdr[0] >> 16);
    // sub-blocks 2g, 2g+1: for g < 2 the 6-bit fields sit in scales[0..7]; for g >= 2 the
    // low 4 bits are in scales[8..11] and the high 2 bits in bits 6-7 of scales[0..7]
    constexpr int sh = 16 * (SUB & 1);
    const uint32_t ws = r.hdr[1] >> sh, wm = r.hdr[2] >> sh, lo = r.hdr[3] >> sh;
    constexpr bool hi = SUB >= 2;
    const int sc0 = hi ? (int)((lo & 15) | (((ws >> 6) & 3) << 4)) : (int)(ws & 63);
    const int sc1 = hi ? (int)(((lo >> 8) & 15) | (((ws >> 14) & 3) << 4)) : (int)((ws >> 8) & 63);
    const int m0 = hi ? (int)(((lo >> 4) & 15) | (((wm >> 6) & 3) << 4)) : (int)(wm & 63);
    const int m1 = hi ? (int)(((lo >> 12) & 15) | (((wm >> 14) & 3) << 4)) : (int)((wm >> 8) & 63);
    const float d1a = d * (float)sc0, m1a = dmin * (float)m0;
    const float d1b = d * (float)sc1, m1b = dmin * (float)m1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = r.q[i >> 1] >> (16 * (i & 1));
      const float l0 = (float)(w & 15), l1 = (float)((w >> 8) & 15);
      const float h0 = (float)((w >> 4) & 15), h1 = (float)((w >> 12) & 15);
      out[i] = f2bf2(__builtin_fmaf(d1a, l0, -m1a), __builtin_fmaf(d1a, l1, -m1a));
      out[8 + i] = f2bf2(__builtin_fmaf(d1b, h0, -m1b), __builtin_fmaf(d1b, h1, -m1b));
    }
  }
  __device__ static int off0(int h) { return 16 * h; }
  __device__ static int off1(int h) { return 32 + 16 * h; }
};

template <>
struct BPiece<GGML_Q8_0> {
  struct Raw { uint32_t w[9]; uint32_t s; };
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  __device__ static int coff(int q) { return 8 * q; }
  template <int SUB>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + (8 * sb + 2 * SUB + h) * QB8_0;
    const uint32_t* a = dword_floor(b);
    r.s = byte_shift(b);  // 0 or 2
    const u32x4_t w0 = gload<u32x4_a4_t>(a), w1 = gload<u32x4_a4_t>(a + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.w[i] = w0[i];
      r.w[4 + i] = w1[i];
    }
    r.w[8] = gload<uint32_t>(a + 8);
  }
  template <int SUB>
  __device__ static void decode(const Raw& r, const uint32_t*, uint32_t out[16]) {
    const float d = half_bits_to_float(r.s ? (r.w[0] >> 16) : (r.w[0] & 0xFFFF));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t q = r.s ? r.w[i + 1] : alignbyte(r.w[i + 1], r.w[i], 2);
      const float y0 = d * (float)(int8_t)(q & 0xFF), y1 = d * (float)(int8_t)((q >> 8) & 0xFF);
      const float y2 = d * (float)(int8_t)((q >> 16) & 0xFF), y3 = d * (float)(int8_t)(q >> 24);
      out[2 * i] = f2bf2(y0, y1);
      out[2 * i + 1] = f2bf2(y2, y3);
    }
  }
  __device__ static int off0(int h) { return 32 * h; }
  __device__ static int off1(int h) { return 32 * h + 16; }
};

template <>
struct BPiece<GGML_Q6_K> {
  struct Raw { uint32_t ql[5], qh[5], sw0, sw1, dw; uint32_t s; uint32_t sp; };
  template <int SUB>
  __device__ static int ksub() { return 128 * (SUB >> 1) + 32 * (SUB & 1); }
  __device__ static int coff(int q) { return q < 4 ? 8 * q : 64 + 8 * (q - 4); }
  template <int SUB>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + sb * QB6_K;
    constexpr int hh = SUB >> 1, c = SUB & 1;
    r.s = byte_shift(b);
    const uint32_t* ql = dword_floor(b + 64 * hh + 32 * c + 16 * h);
    const uint32_t* qh = dword_floor(b + 128 + 32 * hh + 16 * h);
    // 16 bytes each from the dword below them: one dwordx4 and the dword after it
    const u32x4_t l4 = gload<u32x4_a4_t>(ql), h4 = gload<u32x4_a4_t>(qh);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ql[i] = l4[i];
      r.qh[i] = h4[i];
    }
    r.ql[4] = gload<uint32_t>(ql + 4);
    r.qh[4] = gload<uint32_t>(qh + 4);
    // scales[8hh + 2c + h] and scales[8hh + 2c + h + 4] (run c+2) lie in the 8 bytes from
    // the dword below the first
    const uint8_t* sc = b + 192 + 8 * hh + 2 * c + h;
    r.sp = 8 * byte_shift(sc);
    const u32x2_t s2 = gload<u32x2_a4_t>(dword_floor(sc));
    r.sw0 = s2[0];
    r.sw1 = s2[1];
    r.dw = gload<uint32_t>(dword_floor(b + 208));
  }
  template <int SUB>
  __device__ static void decode(const Raw& r, const uint32_t*, uint32_t out[16]) {
    const float d = half_bits_to_float(r.s ? (r.dw >> 16) : (r.dw & 0xFFFF));
    const float d1a = d * (float)(int8_t)((r.sw0 >> r.sp) & 0xFF);
    const float d1b = d * (float)(int8_t)((r.sw1 >> r.sp) & 0xFF);
    constexpr int hsh = 2 * (SUB & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lw = alignbyte(r.ql[i + 1], r.ql[i], r.s);
      const uint32_t hw = alignbyte(r.qh[i + 1], r.qh[i], r.s);
      const uint32_t va = (lw & 0x0F0F0F0Fu) | (((hw >> hsh) & 0x03030303u) << 4);
      const uint32_t vb = ((lw >> 4) & 0x0F0F0F0Fu) | (((hw >> (hsh + 4)) & 0x03030303u) << 4);
      out[2 * i] = f2bf2(d1a * (float)((int)(va & 0xFF) - 32), d1a * (float)((int)((va >> 8) & 0xFF) - 32));
      out[2 * i + 1] = f2bf2(d1a * (float)((int)((va >> 16) & 0xFF) - 32), d1a * (float)((int)(va >> 24) - 32));
      out[8 + 2 * i] = f2bf2(d1b * (float)((int)(vb & 0xFF) - 32), d1b * (float)((int)((vb >> 8) & 0xFF) - 32));
      out[8 + 2 * i + 1] = f2bf2(d1b * (float)((int)((vb >> 16) & 0xFF) - 32), d1b * (float)((int)(vb >> 24) - 32));
    }
  }
  __device__ static int off0(int h) { return 16 * h; }
  __device__ static int off1(int h) { return 32 + 16 * h; }
};

template <>
struct BPiece<GGML_IQ3_S> {
  struct Raw { uint32_t qs0, qs1, sg, misc; };  // misc: d | qh << 16 | scale nibble << 24
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  __device__ static int coff(int q) { return 8 * q; }
  template <int SUB>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + sb * QBIQ3_S;
    const int ib = 2 * SUB + h;
    r.qs0 = ld_u32_a2(b + 2 + 8 * ib);
    r.qs1 = ld_u32_a2(b + 6 + 8 * ib);
    r.sg = ld_u32_a2(b + 74 + 4 * ib);
    const uint32_t nib = (gload<uint8_t>(b + 106 + ib / 2) >> (4 * (ib & 1))) & 15;
    r.misc = (uint32_t)ld_u16(b) | ((uint32_t)gload<uint8_t>(b + 66 + ib) << 16) | (nib << 24);
  }
  template <int SUB>
  __device__ static void decode(const Raw& r, const uint32_t* grid, uint32_t out[16]) {
    const float db = half_bits_to_float(r.misc & 0xFFFF) * (float)(1 + 2 * (int)(r.misc >> 24));
    const uint32_t qh = (r.misc >> 16) & 0xFF;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t sb = (r.sg >> (8 * l)) & 0xFF;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int k = 2 * l + sub;
        const uint32_t qsb = ((k < 4 ? r.qs0 : r.qs1) >> (8 * (k & 3))) & 0xFF;
        const uint32_t g = grid[qsb | (((qh >> k) & 1) << 8)];
        float y[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = db * (float)((g >> (8 * j)) & 0xFF);
          y[j] = ((sb >> (4 * sub + j)) & 1) ? -v : v;
        }
        out[2 * k] = f2bf2(y[0], y[1]);
        out[2 * k + 1] = f2bf2(y[2], y[3]);
      }
    }
  }
  __device__ static int off0(int h) { return 32 * h; }
  __device__ static int off1(int h) { return 32 * h + 16; }
};

}  // namespace ktmi
