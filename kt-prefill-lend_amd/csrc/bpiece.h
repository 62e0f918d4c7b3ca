// B pieces for the grouped MFMA GEMMs: one lane's 32 dequantised weights of one row for
// one 64-value K step, as 16 packed bf16 words.
//
// Each format is split into load_head() (the bytes a super-block column shares over its
// four steps: scales, d), load<SUB>() (the step's quant bytes) and decode() (ALU only), so
// a kernel can keep the loads two steps ahead of their use, load the shared bytes once per
// super-block, and decode after the MFMAs of the previous step. The values are the exact
// dequantisation of formats.h rounded once to bf16 (Q4_K uses an FMA: d*sc*q is exact in
// fp32, so fma(d*sc, q, -dmin*m) rounds the same value as the separate multiply and
// subtract).
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
// Every SUB-dependent member also exists with the step parity as a run-time value: the
// `_hp<S2>(..., p)` forms take SUB = 2 S2 + p with S2 a compile-time constant and p a
// per-lane value (the decode-sized layer's 16x16x32 MFMA operands hold pieces of both
// parities in one wave); the `<SUB>` forms are those with p constant. One body per format
// serves both, so the values are the same.
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

// a & m where the compiler cannot see the mask, so byte extracts of the result stay
// single v_cvt_f32_ubyteN conversions instead of folding into bit-field extracts
__device__ __forceinline__ uint32_t and_opaque(uint32_t a, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(a));
  return r;
}

// (a & m) | (b & ~m) as one v_bfi_b32 (the compiler otherwise spends an AND, an AND and an OR)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(a), "v"(b));
  return r;
}

// (a & m) | b as one v_and_or_b32 (opaque to the compiler, which would otherwise split the
// mask per 16-bit half of a result used as two halves)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
  return r;
}

// Where a piece's bytes are read from: global memory (through the caches) or LDS (rows a
// kernel has staged there, at the same offsets as in the row).
struct GMem {
  template <typename T>
  __device__ __forceinline__ static T ld(const void* p) { return gload<T>(p); }
};
struct LMem {
  // the LDS offset is the generic address's low 32 bits (an address-space cast of a generic
  // pointer would add a null check that the compiler here lowers wrongly)
  template <typename T>
  __device__ __forceinline__ static T ld(const void* p) {
    return *(const __attribute__((address_space(3))) T*)(uintptr_t)(uint32_t)(uintptr_t)p;
  }
};

template <int TYPE>
struct BPiece;

// lookup<SUB>() issues a piece's codebook reads, convert<SUB>() does the rest of decode<SUB>()
// with them (a kernel can put the reads ahead of other LDS traffic). Formats without a
// codebook read nothing there.
template <class P>
struct NoLookup {
  struct Look {};
  template <int SUB, class Head, class Raw>
  __device__ static void lookup(const Head&, const Raw&, const uint32_t*, Look&) {}
  template <int SUB, class Head, class Raw>
  __device__ static void convert(const Head& hd, const Raw& r, const uint32_t* grid, const Look&, uint32_t out[16]) {
    P::template decode<SUB>(hd, r, grid, out);
  }
  template <int S2, class Head, class Raw>
  __device__ static void lookup_hp(const Head&, const Raw&, const uint32_t*, int, Look&) {}
  template <int S2, class Head, class Raw>
  __device__ static void convert_hp(const Head& hd, const Raw& r, const uint32_t* grid, int p, const Look&,
                                    uint32_t out[16]) {
    P::template decode_hp<S2>(hd, r, grid, p, out);
  }
  // the <SUB> forms through the run-time parity bodies
  template <int SUB, class Raw>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t* grid, Raw& r) {
    P::template load_hp<SUB / 2>(row, sb, h, SUB & 1, grid, r);
  }
  template <int SUB, class Head, class Raw>
  __device__ static void decode(const Head& hd, const Raw& r, const uint32_t* grid, uint32_t out[16]) {
    P::template decode_hp<SUB / 2>(hd, r, grid, SUB & 1, out);
  }
  // load<SUB> for a kernel that holds the raw bytes of step SUB - 1 of the same super-block
  // in `prev` (a format whose step pairs share bytes takes them from there)
  template <int SUB, class Raw>
  __device__ static void load_next(const uint8_t* row, int sb, int h, const uint32_t* grid, Raw& r, const Raw&) {
    P::template load_hp<SUB / 2>(row, sb, h, SUB & 1, grid, r);
  }
};

template <>
struct BPiece<GGML_Q4_K> : NoLookup<BPiece<GGML_Q4_K>> {
  static constexpr int NLOAD = 1;  // VMEM instructions per load<SUB>, at least
  static constexpr int NLOAD2 = 2;  // VMEM instructions of load_next over two consecutive steps
  static constexpr int VPM = 4;    // VALU instructions the GEMM schedule places after each MFMA
  struct Head { u32x4_t hdr; };  // d, dmin, scales[12]
  struct Raw { u32x4_t q; };
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  template <int S2>
  __device__ static int ksub_hp(int p) { return 128 * S2 + 64 * p; }
  __device__ static int coff(int q) { return 8 * q; }
  template <class M = GMem>
  __device__ static void load_head(const uint8_t* row, int sb, int, Head& hd) { hd.hdr = M::template ld<u32x4_t>(row + sb * QB4_K); }
  template <int S2, class M = GMem>
  __device__ __forceinline__ static void load_hp(const uint8_t* row, int sb, int h, int p, const uint32_t*, Raw& r) {
    r.q = M::template ld<u32x4_t>(row + sb * QB4_K + 16 + 64 * S2 + 32 * p + 16 * h);
  }
  template <int S2>
  __device__ __forceinline__ static void decode_hp(const Head& hd, const Raw& r, const uint32_t*, int p,
                                                   uint32_t out[16]) {
    const float d = half_bits_to_float(hd.hdr[0] & 0xFFFF);
    const float dmin = half_bits_to_float(hd.hdr[0] >> 16);
    // sub-blocks 2g, 2g+1 (g = SUB = 2 S2 + p): for g < 2 the 6-bit fields sit in
    // scales[0..7]; for g >= 2 the low 4 bits are in scales[8..11] and the high 2 bits in
    // bits 6-7 of scales[0..7]
    const int sh = 16 * p;
    const uint32_t ws = hd.hdr[1] >> sh, wm = hd.hdr[2] >> sh, lo = hd.hdr[3] >> sh;
    constexpr bool hi = S2 == 1;
    const int sc0 = hi ? (int)((lo & 15) | (((ws >> 6) & 3) << 4)) : (int)(ws & 63);
    const int sc1 = hi ? (int)(((lo >> 8) & 15) | (((ws >> 14) & 3) << 4)) : (int)((ws >> 8) & 63);
    const int m0 = hi ? (int)(((lo >> 4) & 15) | (((wm >> 6) & 3) << 4)) : (int)(wm & 63);
    const int m1 = hi ? (int)(((lo >> 12) & 15) | (((wm >> 14) & 3) << 4)) : (int)((wm >> 8) & 63);
    const float d1a = d * (float)sc0, m1a = dmin * (float)m0;
    const float d1b = d * (float)sc1, m1b = dmin * (float)m1;
    // 4 bytes = 4 low nibbles (positions off0..) and 4 high nibbles (off1..); each nibble
    // masked into its own byte converts with one v_cvt_f32_ubyteN
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t nl = and_opaque(r.q[i], 0x0F0F0F0Fu), nh = and_opaque(r.q[i] >> 4, 0x0F0F0F0Fu);
      out[2 * i] = f2bf2(__builtin_fmaf(d1a, (float)(nl & 0xFF), -m1a), __builtin_fmaf(d1a, (float)((nl >> 8) & 0xFF), -m1a));
      out[2 * i + 1] = f2bf2(__builtin_fmaf(d1a, (float)((nl >> 16) & 0xFF), -m1a), __builtin_fmaf(d1a, (float)(nl >> 24), -m1a));
      out[8 + 2 * i] = f2bf2(__builtin_fmaf(d1b, (float)(nh & 0xFF), -m1b), __builtin_fmaf(d1b, (float)((nh >> 8) & 0xFF), -m1b));
      out[8 + 2 * i + 1] = f2bf2(__builtin_fmaf(d1b, (float)((nh >> 16) & 0xFF), -m1b), __builtin_fmaf(d1b, (float)(nh >> 24), -m1b));
    }
  }
  __device__ static int off0(int h) { return 16 * h; }
  __device__ static int off1(int h) { return 32 + 16 * h; }
};

template <>
struct BPiece<GGML_Q8_0> : NoLookup<BPiece<GGML_Q8_0>> {
  static constexpr int NLOAD = 3;  // VMEM instructions per load<SUB>, at least
  static constexpr int NLOAD2 = 6;  // VMEM instructions of load_next over two consecutive steps
  static constexpr int VPM = 4;    // VALU instructions the GEMM schedule places after each MFMA
  struct Head {};
  struct Raw { uint32_t w[9]; uint32_t s; };
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  template <int S2>
  __device__ static int ksub_hp(int p) { return 128 * S2 + 64 * p; }
  __device__ static int coff(int q) { return 8 * q; }
  template <class M = GMem>
  __device__ static void load_head(const uint8_t*, int, int, Head&) {}
  template <int S2, class M = GMem>
  __device__ __forceinline__ static void load_hp(const uint8_t* row, int sb, int h, int p, const uint32_t*, Raw& r) {
    const uint8_t* b = row + (8 * sb + 4 * S2 + 2 * p + h) * QB8_0;
    const uint32_t* a = dword_floor(b);
    r.s = byte_shift(b);  // 0 or 2
    const u32x4_t w0 = M::template ld<u32x4_a4_t>(a), w1 = M::template ld<u32x4_a4_t>(a + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.w[i] = w0[i];
      r.w[4 + i] = w1[i];
    }
    r.w[8] = M::template ld<uint32_t>(a + 8);
  }
  template <int S2>
  __device__ __forceinline__ static void decode_hp(const Head&, const Raw& r, const uint32_t*, int, uint32_t out[16]) {
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
struct BPiece<GGML_Q6_K> : NoLookup<BPiece<GGML_Q6_K>> {
  static constexpr int NLOAD = 4;  // VMEM instructions per load<SUB>, at least
  // VMEM instructions of load_next over two consecutive steps: the odd step of a pair loads
  // only its ql bytes (the pair's qh bytes are the same)
  static constexpr int NLOAD2 = 6;
  // VALU instructions the GEMM schedule places after each MFMA: 4 for a decode of 4.1 a MFMA
  // (headline down GEMM 255 -> 250 us at the sustained clock; 5 and 6 slower, 3 no better)
  static constexpr int VPM = 4;
  // the 20 bytes from the dword below scales[0]: scales[16] and d, s = byte shift
  struct Head { uint32_t w[5]; uint32_t s; };
  struct Raw { uint32_t ql[5], qh[5]; };
  template <int SUB>
  __device__ static int ksub() { return 128 * (SUB >> 1) + 32 * (SUB & 1); }
  template <int S2>
  __device__ static int ksub_hp(int p) { return 128 * S2 + 32 * p; }
  __device__ static int coff(int q) { return q < 4 ? 8 * q : 64 + 8 * (q - 4); }
  template <class M = GMem>
  __device__ static void load_head(const uint8_t* row, int sb, int, Head& hd) {
    const uint8_t* sc = row + sb * QB6_K + 192;
    hd.s = byte_shift(sc);
    const uint32_t* a = dword_floor(sc);
    const u32x4_t w = M::template ld<u32x4_a4_t>(a);
#pragma unroll
    for (int i = 0; i < 4; ++i) hd.w[i] = w[i];
    hd.w[4] = M::template ld<uint32_t>(a + 4);
  }
  template <int S2, class M = GMem>
  __device__ __forceinline__ static void load_hp(const uint8_t* row, int sb, int h, int p, const uint32_t*, Raw& r) {
    const uint8_t* b = row + sb * QB6_K;
    constexpr int hh = S2;
    const int c = p;
    const uint32_t* ql = dword_floor(b + 64 * hh + 32 * c + 16 * h);
    const uint32_t* qh = dword_floor(b + 128 + 32 * hh + 16 * h);
    // 16 bytes each from the dword below them: one dwordx4 and the dword after it
    const u32x4_t l4 = M::template ld<u32x4_a4_t>(ql), h4 = M::template ld<u32x4_a4_t>(qh);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ql[i] = l4[i];
      r.qh[i] = h4[i];
    }
    r.ql[4] = M::template ld<uint32_t>(ql + 4);
    r.qh[4] = M::template ld<uint32_t>(qh + 4);
  }
  // steps 2 hh and 2 hh + 1 read the same 16 qh bytes (bits 2c.. of run c, c = SUB & 1): the
  // odd step takes them from the even one's raw bytes and loads only its ql bytes
  template <int SUB>
  __device__ __forceinline__ static void load_next(const uint8_t* row, int sb, int h, const uint32_t* grid, Raw& r,
                                                   const Raw& prev) {
    if constexpr ((SUB & 1) == 0) {
      load_hp<SUB / 2>(row, sb, h, 0, grid, r);
    } else {
      const uint32_t* ql = dword_floor(row + sb * QB6_K + 64 * (SUB / 2) + 32 + 16 * h);
      const u32x4_t l4 = GMem::ld<u32x4_a4_t>(ql);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.ql[i] = l4[i];
      r.ql[4] = GMem::ld<uint32_t>(ql + 4);
#pragma unroll
      for (int i = 0; i < 5; ++i) r.qh[i] = prev.qh[i];
    }
  }
  template <int S2>
  __device__ __forceinline__ static void decode_hp(const Head& hd, const Raw& r, const uint32_t*, int p,
                                                   uint32_t out[16]) {
    constexpr int hh = S2;
    const int c = p;
    const uint32_t s = hd.s;  // the same shift as the block start (192 = 0 mod 4)
    // scales[8hh + 2c + h] (run c) and scales[8hh + 2c + h + 4] (run c+2): bytes 2c + h of
    // the realigned scale words 2hh and 2hh + 1
    const uint32_t h8 = 8 * ((threadIdx.x >> 5) & 1);
    const uint32_t sa = alignbyte(hd.w[2 * hh + 1], hd.w[2 * hh], s);
    const uint32_t sbw = alignbyte(hd.w[2 * hh + 2], hd.w[2 * hh + 1], s);
    const float d = half_bits_to_float(alignbyte(hd.w[4], hd.w[4], s) & 0xFFFF);
    // y = (d sc) (q - 32) as the product of (d sc / 4), exact, and the signed byte 4 (q - 32),
    // converted with one v_cvt_f32_i32 (sdwa, sign-extended byte): one rounding of the exact
    // product, and the signed zeros of a plain multiply (q = 32 under a negative scale
    // gives -0, as (d sc) * 0 does). The 6-bit code q - 32 is q with its bit 5 flipped, read
    // as 6-bit two's complement: flipping bits 1, 3, 5, 7 of every qh byte flips bit 5 of
    // both runs' codes; the code then sits in bits 2..7 of its byte.
    const float d1a = 0.25f * (d * (float)(int8_t)((sa >> (16 * c + h8)) & 0xFF));
    const float d1b = 0.25f * (d * (float)(int8_t)((sbw >> (16 * c + h8)) & 0xFF));
    const int hsh = 2 * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lw = alignbyte(r.ql[i + 1], r.ql[i], s);
      const uint32_t hw = alignbyte(r.qh[i + 1], r.qh[i], s) ^ 0xAAAAAAAAu;
      // run c: low nibbles and qh bits hsh, hsh+1; run c+2: high nibbles and bits hsh+4, hsh+5
      const uint32_t va = bfi(0xC0C0C0C0u, hw << (6 - hsh), (lw & 0x0F0F0F0Fu) << 2);
      const uint32_t vb = bfi(0xC0C0C0C0u, hw << (2 - hsh), (lw >> 2) & 0x3C3C3C3Cu);
      out[2 * i] = f2bf2(d1a * (float)(int8_t)(va & 0xFF), d1a * (float)(int8_t)((va >> 8) & 0xFF));
      out[2 * i + 1] = f2bf2(d1a * (float)(int8_t)((va >> 16) & 0xFF), d1a * (float)(int8_t)(va >> 24));
      out[8 + 2 * i] = f2bf2(d1b * (float)(int8_t)(vb & 0xFF), d1b * (float)(int8_t)((vb >> 8) & 0xFF));
      out[8 + 2 * i + 1] = f2bf2(d1b * (float)(int8_t)((vb >> 16) & 0xFF), d1b * (float)(int8_t)(vb >> 24));
    }
  }
  __device__ static int off0(int h) { return 16 * h; }
  __device__ static int off1(int h) { return 32 + 16 * h; }
};

template <>
struct BPiece<GGML_IQ3_S> {
  // `grid` is the codebook as byte selectors, staged in LDS by stage_iq3s_sel (formats.h).
  // VMEM instructions per load<SUB>: qs (dwordx2 + dword, merged into one dwordx3), the
  // signs (dwordx2) and the qh dword
  static constexpr int NLOAD = 3;
  static constexpr int NLOAD2 = 6;  // VMEM instructions of load_next over two consecutive steps
  static constexpr int VPM = 4;    // VALU instructions the GEMM schedule places after each MFMA
  // d and the 4 scale bytes of the block (dwords below them, realigned at decode)
  struct Head { uint32_t dw, sc0, sc1; uint32_t s; };
  // qs[8] of group ib (3 dwords from below), qh byte's dword, signs[4] (2 dwords from below)
  struct Raw { uint32_t qs[3], sg[2], qh; };
  template <int SUB>
  __device__ static int ksub() { return 64 * SUB; }
  template <int S2>
  __device__ static int ksub_hp(int p) { return 128 * S2 + 64 * p; }
  __device__ static int coff(int q) { return 8 * q; }
  template <class M = GMem>
  __device__ static void load_head(const uint8_t* row, int sb, int, Head& hd) {
    const uint8_t* b = row + sb * QBIQ3_S;
    hd.s = byte_shift(b);
    hd.dw = M::template ld<uint32_t>(dword_floor(b));
    hd.sc0 = M::template ld<uint32_t>(dword_floor(b + 106));
    hd.sc1 = M::template ld<uint32_t>(dword_floor(b + 108));
  }
  template <int S2, class M = GMem>
  __device__ __forceinline__ static void load_hp(const uint8_t* row, int sb, int h, int p, const uint32_t*, Raw& r) {
    const uint8_t* b = row + sb * QBIQ3_S;
    const int ib = 4 * S2 + 2 * p + h;
    const uint32_t* q = dword_floor(b + 2 + 8 * ib);
    const u32x2_t q2 = M::template ld<u32x2_a4_t>(q);
    r.qs[0] = q2[0];
    r.qs[1] = q2[1];
    r.qs[2] = M::template ld<uint32_t>(q + 2);
    const u32x2_t s2 = M::template ld<u32x2_a4_t>(dword_floor(b + 74 + 4 * ib));
    r.sg[0] = s2[0];
    r.sg[1] = s2[1];
    r.qh = M::template ld<uint32_t>(dword_floor(b + 66 + ib));
  }
  // the 8 codebook entries of the piece's 4-value groups
  struct Look { uint32_t g[8]; };
  template <int S2>
  __device__ __forceinline__ static void lookup_hp(const Head& hd, const Raw& r, const uint32_t* grid, int p,
                                                   Look& lk) {
    const uint32_t s = hd.s;
    const uint32_t h = (threadIdx.x >> 5) & 1;
    const int ib = 4 * S2 + 2 * p + (int)h;
    // block byte offsets: qs at 2 + 8 ib (= s + 2 mod 4), qh at 66 + ib
    const uint32_t s2 = (s + 2) & 3;
    const uint32_t qs0 = alignbyte(r.qs[1], r.qs[0], s2), qs1 = alignbyte(r.qs[2], r.qs[1], s2);
    const uint32_t qh = __builtin_amdgcn_ubfe(r.qh, 8 * ((s + 2 + ib) & 3), 8);
    const uint32_t qh2 = qh | (qh << 16);
    // the 9-bit indices of groups 2j and 2j + 1 as the two 16-bit halves of one word: their
    // qs bytes moved to bits 0 and 16 by one v_perm, qh bits 2j and 2j + 1 to bits 8 and 24
    // by one packed 16-bit shift of qh2 and merged with one v_and_or; each half then becomes
    // an LDS address with one v_lshlrev_b32_sdwa (2.5 VALU an index instead of 4)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t qsw = j < 2 ? qs0 : qs1;
      const uint32_t b0 = (2 * j) & 3, b1 = (2 * j + 1) & 3;
      const uint32_t lo = __builtin_amdgcn_perm(0u, qsw, b0 | 0x0C00u | (b1 << 16) | 0x0C000000u);
      const u16x2_t hv = __builtin_bit_cast(u16x2_t, qh2) << u16x2_t{(uint16_t)(8 - 2 * j), (uint16_t)(7 - 2 * j)};
      const uint32_t w = and_or(__builtin_bit_cast(uint32_t, hv), 0x01000100u, lo);
      lk.g[2 * j] = grid[w & 0xFFFF];
      lk.g[2 * j + 1] = grid[w >> 16];
    }
  }
  template <int S2>
  __device__ __forceinline__ static void convert_hp(const Head& hd, const Raw& r, const uint32_t*, int p,
                                                    const Look& lk, uint32_t out[16]) {
    const uint32_t s = hd.s;
    const uint32_t h = (threadIdx.x >> 5) & 1;
    const int ib = 4 * S2 + 2 * p + (int)h;
    // block byte offsets: signs at 74 + 4 ib (= s + 2 mod 4), scales at 106, d at 0
    const uint32_t s2 = (s + 2) & 3;
    const uint32_t sg = alignbyte(r.sg[1], r.sg[0], s2);
    const uint32_t scw = alignbyte(hd.sc1, hd.sc0, s2);  // scales[0..3]
    const uint32_t nib = (scw >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15;
    const uint32_t dbits = (hd.dw >> (8 * s)) & 0xFFFF;
    const float db = half_bits_to_float(dbits) * (float)(1 + 2 * (int)nib);
    // A group has only eight magnitudes m = 2e + 1: bf16(db * m) of each (the same rounding
    // of the same exact product as a value-by-value decode) goes into a table of two byte
    // planes, byte e of {tl1:tl0} the low byte of entry e, of {th1:th0} its high byte. The
    // codebook entries are staged as selectors e (stage_iq3s_sel), so one v_perm per plane
    // gathers the four values of a codebook entry and two more interleave them into bf16
    // pairs: 8 VALU per four values with the signs, against 14 for convert, scale and pack.
    uint32_t pw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pw[i] = f2bf2(db * (float)(4 * i + 1), db * (float)(4 * i + 3));
    const uint32_t tl0 = __builtin_amdgcn_perm(pw[1], pw[0], 0x06040200u);
    const uint32_t th0 = __builtin_amdgcn_perm(pw[1], pw[0], 0x07050301u);
    const uint32_t tl1 = __builtin_amdgcn_perm(pw[3], pw[2], 0x06040200u);
    const uint32_t th1 = __builtin_amdgcn_perm(pw[3], pw[2], 0x07050301u);
    // value 4k + j takes sign bit 4k + j of sg. (sign ? -v : v) of v = db * m flips the sign
    // bit of v, and so of its bf16 rounding: bits 2p and 2p + 1 of sg are moved to bits 15
    // and 31 of the packed pair of values 2p, 2p + 1 by one packed 16-bit shift of sg's
    // half-word (in both halves) and xored in
    const uint32_t sgw[2] = {(sg & 0xFFFFu) | (sg << 16), (sg >> 16) | (sg & 0xFFFF0000u)};
    auto pair_signs = [&](int pr) {
      const int q = (2 * pr) & 15;
      const u16x2_t v = __builtin_bit_cast(u16x2_t, sgw[pr >> 3]) << u16x2_t{(uint16_t)(15 - q), (uint16_t)(14 - q)};
      return __builtin_bit_cast(uint32_t, v) & 0x80008000u;
    };
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t lo = __builtin_amdgcn_perm(tl1, tl0, lk.g[k]);  // low bytes of values 0..3
      const uint32_t hi = __builtin_amdgcn_perm(th1, th0, lk.g[k]);  // their high bytes
      out[2 * k] = __builtin_amdgcn_perm(hi, lo, 0x05010400u) ^ pair_signs(2 * k);
      out[2 * k + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u) ^ pair_signs(2 * k + 1);
    }
  }
  template <int S2>
  __device__ __forceinline__ static void decode_hp(const Head& hd, const Raw& r, const uint32_t* grid, int p,
                                                   uint32_t out[16]) {
    Look lk;
    lookup_hp<S2>(hd, r, grid, p, lk);
    convert_hp<S2>(hd, r, grid, p, lk, out);
  }
  // the <SUB> forms through the run-time parity bodies
  template <int SUB>
  __device__ static void load(const uint8_t* row, int sb, int h, const uint32_t* grid, Raw& r) {
    load_hp<SUB / 2>(row, sb, h, SUB & 1, grid, r);
  }
  template <int SUB>
  __device__ static void load_next(const uint8_t* row, int sb, int h, const uint32_t* grid, Raw& r, const Raw&) {
    load_hp<SUB / 2>(row, sb, h, SUB & 1, grid, r);
  }
  template <int SUB>
  __device__ static void lookup(const Head& hd, const Raw& r, const uint32_t* grid, Look& lk) {
    lookup_hp<SUB / 2>(hd, r, grid, SUB & 1, lk);
  }
  template <int SUB>
  __device__ static void convert(const Head& hd, const Raw& r, const uint32_t* grid, const Look& lk, uint32_t out[16]) {
    convert_hp<SUB / 2>(hd, r, grid, SUB & 1, lk, out);
  }
  template <int SUB>
  __device__ static void decode(const Head& hd, const Raw& r, const uint32_t* grid, uint32_t out[16]) {
    decode_hp<SUB / 2>(hd, r, grid, SUB & 1, out);
  }
  __device__ static int off0(int h) { return 32 * h; }
  __device__ static int off1(int h) { return 32 * h + 16; }
};

}  // namespace ktmi
