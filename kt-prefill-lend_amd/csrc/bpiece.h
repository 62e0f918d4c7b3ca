// B-tile pieces for the grouped MFMA GEMMs: one thread's 32 dequantised weights of one
// row for one 64-value K step, as 16 packed bf16 words.
//
// Each format is split into load() (global loads only, into registers) and decode()
// (ALU only), so a kernel can issue the loads of step k+1 before the MFMAs of step k and
// decode after them. The values are the exact dequantisation of formats.h rounded once
// to bf16 (Q4_K uses an FMA: d*sc*q is exact in fp32, so fma(d*sc, q, -dmin*m) rounds the
// same value as the separate multiply and subtract).
//
// Piece h (0 or 1) of the K step starting at k0 (a multiple of 64) covers:
//   Q4_K : values [16h, 16h+16) and [32+16h, 32+16h+16): the two nibbles of qs bytes
//          [32g+16h, +16), g = (k0 % 256) / 64 (sub-blocks 2g and 2g+1)
//   others: values [32h, 32h+32) (one Q8_0 block, one Q6_K 32-run, one IQ3_S group)
// `off0`/`off1` give the K-step offsets of out[0..7] and out[8..15] (16 values each).
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
  struct Raw { u32x4_t hdr, q; int g; };
  __device__ static void load(const uint8_t* row, int k0, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + (k0 >> 8) * QB4_K;
    r.g = (k0 & 255) >> 6;
    r.hdr = *(const u32x4_t*)b;
    r.q = *(const u32x4_t*)(b + 16 + 32 * r.g + 16 * h);
  }
  __device__ static void decode(const Raw& r, const uint32_t*, uint32_t out[16]) {
    const float d = half_bits_to_float(r.hdr[0] & 0xFFFF);
    const float dmin = half_bits_to_float(r.hdr[0] >> 16);
    int sc0, sc1, m0, m1;
    if (r.g < 2) {  // sub-blocks 2g, 2g+1 < 4: 6-bit fields in scales[0..7]
      const uint32_t ws = r.hdr[1] >> (16 * r.g), wm = r.hdr[2] >> (16 * r.g);
      sc0 = ws & 63;
      sc1 = (ws >> 8) & 63;
      m0 = wm & 63;
      m1 = (wm >> 8) & 63;
    } else {  // sub-blocks 4..7: low 4 bits in scales[8..11], high 2 bits in bits 6-7 of scales[0..7]
      const int sh = 16 * (r.g - 2);
      const uint32_t lo = r.hdr[3] >> sh, hs = r.hdr[1] >> sh, hm = r.hdr[2] >> sh;
      sc0 = (lo & 15) | (((hs >> 6) & 3) << 4);
      sc1 = ((lo >> 8) & 15) | (((hs >> 14) & 3) << 4);
      m0 = ((lo >> 4) & 15) | (((hm >> 6) & 3) << 4);
      m1 = ((lo >> 12) & 15) | (((hm >> 14) & 3) << 4);
    }
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
  __device__ static void load(const uint8_t* row, int k0, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + ((k0 >> 5) + h) * QB8_0;
    const uint32_t* a = dword_floor(b);
    r.s = byte_shift(b);  // 0 or 2
#pragma unroll
    for (int i = 0; i < 9; ++i) r.w[i] = a[i];
  }
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
  struct Raw { uint32_t ql[9], qh[9], sw, dw; uint32_t s; int c; };
  __device__ static void load(const uint8_t* row, int k0, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + (k0 >> 8) * QB6_K;
    const int e0 = (k0 & 255) + 32 * h;
    const int hh = e0 >> 7;
    r.c = (e0 & 127) >> 5;
    r.s = byte_shift(b);
    const uint32_t* ql = dword_floor(b + 64 * hh + 32 * (r.c & 1));
    const uint32_t* qh = dword_floor(b + 128 + 32 * hh);
#pragma unroll
    for (int i = 0; i < 9; ++i) {
      r.ql[i] = ql[i];
      r.qh[i] = qh[i];
    }
    r.sw = *dword_floor(b + 192 + 8 * hh + 2 * r.c);
    r.dw = *dword_floor(b + 208);
  }
  __device__ static void decode(const Raw& r, const uint32_t*, uint32_t out[16]) {
    const float d = half_bits_to_float(r.s ? (r.dw >> 16) : (r.dw & 0xFFFF));
    const uint32_t sp = 8 * ((r.s + 2 * r.c) & 3);  // byte position of scales[8hh + 2c] in sw
    const float d1a = d * (float)(int8_t)((r.sw >> sp) & 0xFF);
    const float d1b = d * (float)(int8_t)((r.sw >> (sp + 8)) & 0xFF);
    const int lsh = (r.c < 2) ? 0 : 4, hsh = 2 * r.c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lw = alignbyte(r.ql[i + 1], r.ql[i], r.s);
      const uint32_t hw = alignbyte(r.qh[i + 1], r.qh[i], r.s);
      const uint32_t v = ((lw >> lsh) & 0x0F0F0F0Fu) | (((hw >> hsh) & 0x03030303u) << 4);
      const float dd = (i < 4) ? d1a : d1b;
      const float y0 = dd * (float)((int)(v & 0xFF) - 32), y1 = dd * (float)((int)((v >> 8) & 0xFF) - 32);
      const float y2 = dd * (float)((int)((v >> 16) & 0xFF) - 32), y3 = dd * (float)((int)(v >> 24) - 32);
      out[2 * i] = f2bf2(y0, y1);
      out[2 * i + 1] = f2bf2(y2, y3);
    }
  }
  __device__ static int off0(int h) { return 32 * h; }
  __device__ static int off1(int h) { return 32 * h + 16; }
};

template <>
struct BPiece<GGML_IQ3_S> {
  struct Raw { uint32_t qs0, qs1, sg, misc; };  // misc: d | qh << 16 | scale nibble << 24
  __device__ static void load(const uint8_t* row, int k0, int h, const uint32_t*, Raw& r) {
    const uint8_t* b = row + (k0 >> 8) * QBIQ3_S;
    const int ib = ((k0 & 255) >> 5) + h;
    r.qs0 = ld_u32_a2(b + 2 + 8 * ib);
    r.qs1 = ld_u32_a2(b + 6 + 8 * ib);
    r.sg = ld_u32_a2(b + 74 + 4 * ib);
    const uint32_t nib = (b[106 + ib / 2] >> (4 * (ib & 1))) & 15;
    r.misc = (uint32_t)ld_u16(b) | ((uint32_t)b[66 + ib] << 16) | (nib << 24);
  }
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
