// Per-type int8 dot-product units of the GGUF GEMVs (wave64), shared by the decode-window
// GEMV (gemv.hip) and the fused decode layer (decode_layer.hip).
//
// A "unit" is the weight span one lane decodes per step -- 64 values for Q4_K/Q6_K (32
// bytes of packed nibbles shared by two sub-blocks), 32 values for Q8_0/IQ3_S. The
// integer sums equal the reference's vec_dot sums (hot/kt_gguf_moe_multi/vecdotq.cuh
// :969-983 Q8_0, :1326-1367 Q4_K, :1625-1648 Q6_K, :1875-1899 IQ3_S); only the fp32 order
// of the per-block scale products differs.
#pragma once
#include "formats.h"

namespace ktmi {
namespace gemv {

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// q8_1 data of one unit for one member: NQ blocks of 32 int8 + their fp16 d.
template <int NQ>
struct Act {
  uint32_t q[8 * NQ];
  float d[NQ];
  int s[2 * NQ];  // integer sums of the int8 values per 16 (Q6_K) or per 32 (Q4_K, s[0..NQ))
};

template <int NQ>
__device__ __forceinline__ void load_act(const uint8_t* xrow, int ub0, int ub1, Act<NQ>& a) {
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const uint8_t* b = xrow + (int64_t)(j == 0 ? ub0 : ub1) * QB8_1;
    const uint32_t ds = *(const uint32_t*)b;
    a.d[j] = half_bits_to_float(ds & 0xFFFF);
    const u32x4_t v0 = *(const u32x4_a4_t*)(b + 4);  // 36-byte blocks: 4-byte aligned only
    const u32x4_t v1 = *(const u32x4_a4_t*)(b + 20);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a.q[8 * j + i] = v0[i];
      a.q[8 * j + 4 + i] = v1[i];
    }
  }
}

// ---- per-type weight units. load() only issues global loads (wide, from the dword at or
// below each field: the 2-byte aligned formats are realigned with v_alignbyte); finish()
// unpacks them once they have landed, so a thread can put several units' loads in flight
// before it waits for any.

__device__ __forceinline__ const uint32_t* dw_floor(const uint8_t* p) {
  return (const uint32_t*)((uintptr_t)p & ~(uintptr_t)3);
}
__device__ __forceinline__ uint32_t dw_shift(const uint8_t* p) { return (uint32_t)((uintptr_t)p & 3); }
// 8 dwords of the bytes from `sh` into the 9 dwords r[0..8] (sh in {0, 2})
__device__ __forceinline__ void realign8(const uint32_t* r, uint32_t sh, uint32_t* out) {
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], sh);
}
// 9 dwords from the dword-aligned p: two dwordx4 and a dword
__device__ __forceinline__ void load9(const uint32_t* p, uint32_t* r) {
  const u32x4_t a = gload<u32x4_a4_t>(p), b = gload<u32x4_a4_t>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = a[i];
    r[4 + i] = b[i];
  }
  r[8] = gload<uint32_t>(p + 8);
}

template <int TYPE>
struct Unit;

// Q8_0: unit = block u (32 values, 34 bytes: fp16 d, 32 int8)
template <>
struct Unit<GGML_Q8_0> {
  static constexpr int VALS = 32, NQ = 1;
  static constexpr int NLD = 3;  // VMEM instructions of load(), at least (a waitcnt counts on it)
  struct W { uint32_t r[9]; uint32_t sh; uint32_t q[8]; float d; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)u * QB8_0;
    w.sh = dw_shift(b);  // 0 or 2
    load9(dw_floor(b), w.r);
  }
  __device__ static void finish(W& w, const uint32_t*) {
    w.d = half_bits_to_float(w.sh ? (w.r[0] >> 16) : (w.r[0] & 0xFFFF));
    // qs start 2 bytes after the block: byte 2 (sh = 0) or byte 4 (sh = 2) of the dwords
#pragma unroll
    for (int i = 0; i < 8; ++i) w.q[i] = w.sh ? w.r[i + 1] : __builtin_amdgcn_alignbyte(w.r[i + 1], w.r[i], 2);
  }
  __device__ static void qblocks(int u, int& ub0, int& ub1) { ub0 = ub1 = u; }
  __device__ static void prep(Act<1>&) {}
  __device__ static float dot(const W& w, const Act<1>& a) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = dot4(w.q[i], a.q[i], s);
    return w.d * a.d[0] * (float)s;
  }
};

// Q4_K: unit u -> super-block u/4, g = u%4: sub-blocks 2g (low nibbles of qs[32g..32g+32))
// and 2g+1 (high nibbles of the same bytes). Blocks are 16-byte aligned (144 bytes).
template <>
struct Unit<GGML_Q4_K> {
  static constexpr int VALS = 64, NQ = 2;
  static constexpr int NLD = 3;  // VMEM instructions of load(), at least (a waitcnt counts on it)
  struct W { u32x4_t h0; uint32_t q[8]; int g; float d, dmin; int sc0, m0, sc1, m1; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 2) * QB4_K;
    w.g = u & 3;
    w.h0 = gload<u32x4_t>(b);  // d, dmin, scales[12]
    const u32x4_t v0 = gload<u32x4_t>(b + 16 + 32 * w.g);
    const u32x4_t v1 = gload<u32x4_t>(b + 32 + 32 * w.g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w.q[i] = v0[i];
      w.q[4 + i] = v1[i];
    }
  }
  // 6-bit scale and min of sub-block j = 2g + k (k = 0, 1) from the 12 scale bytes in words
  // w1 (bytes 0-3), w2 (4-7), w3 (8-11): j < 4: scales[j] & 63 and scales[j+4] & 63;
  // j >= 4: low 4 bits from scales[j+4], high 2 bits from bits 6-7 of scales[j-4] (scale)
  // and scales[j] (min). Shifts and selects only, for a runtime g.
  __device__ static void scale_min(uint32_t w1, uint32_t w2, uint32_t w3, int j, int& sc, int& m) {
    const uint32_t sh = 8 * (j & 3);
    const uint32_t b1 = (w1 >> sh) & 0xFF, b2 = (w2 >> sh) & 0xFF, b3 = (w3 >> sh) & 0xFF;
    const int lo_sc = (int)(b1 & 63), lo_m = (int)(b2 & 63);
    const int hi_sc = (int)((b3 & 15) | ((b1 >> 6) << 4));
    const int hi_m = (int)((b3 >> 4) | ((b2 >> 6) << 4));
    sc = j < 4 ? lo_sc : hi_sc;
    m = j < 4 ? lo_m : hi_m;
  }
  __device__ static void finish(W& w, const uint32_t*) {
    w.d = half_bits_to_float(w.h0[0] & 0xFFFF);
    w.dmin = half_bits_to_float(w.h0[0] >> 16);
    scale_min(w.h0[1], w.h0[2], w.h0[3], 2 * w.g, w.sc0, w.m0);
    scale_min(w.h0[1], w.h0[2], w.h0[3], 2 * w.g + 1, w.sc1, w.m1);
  }
  __device__ static void qblocks(int u, int& ub0, int& ub1) {
    ub0 = 8 * (u >> 2) + 2 * (u & 3);
    ub1 = ub0 + 1;
  }
  __device__ static void prep(Act<2>& a) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int s = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) s = dot4(0x01010101u, a.q[8 * j + i], s);
      a.s[j] = s;
    }
  }
  __device__ static float dot(const W& w, const Act<2>& a) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s0 = dot4(w.q[i] & 0x0F0F0F0Fu, a.q[i], s0);
      s1 = dot4((w.q[i] >> 4) & 0x0F0F0F0Fu, a.q[8 + i], s1);
    }
    const float sd = a.d[0] * (float)(s0 * w.sc0) + a.d[1] * (float)(s1 * w.sc1);
    const float sm = a.d[0] * (float)(a.s[0] * w.m0) + a.d[1] * (float)(a.s[1] * w.m1);
    return w.d * sd - w.dmin * sm;
  }
};

// Q6_K: unit u -> super-block u/4, v = u%4, h = v/2, c = v%2: values 128h+32c+[0,32) (low
// nibbles of ql[64h+32c..+32), qh bits 2c) and 128h+32(c+2)+[0,32) (high nibbles, qh bits
// 2c+4). q = (nib | hi << 4) - 32 is summed as sum(b*x) - 32*sum(x) with b in 0..63.
// Blocks are 210 bytes: 2-byte aligned.
template <>
struct Unit<GGML_Q6_K> {
  static constexpr int VALS = 64, NQ = 2;
  static constexpr int NLD = 8;  // VMEM instructions of load(), at least (a waitcnt counts on it)
  struct W {
    uint32_t rl[9], rh[9], rs[2], rd;
    uint32_t shq, shs, shd;
    int c;
    uint32_t ql[8], qh[8];
    float d;
    int sc[4];
  };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 2) * QB6_K;
    const int v = u & 3, h = v >> 1;
    w.c = v & 1;
    const uint8_t* pl = b + 64 * h + 32 * w.c;
    const uint8_t* ph = b + 128 + 32 * h;
    const uint8_t* ps = b + 192 + 8 * h + 2 * w.c;  // scales[8h + 2c], +1, +4, +5
    const uint8_t* pd = b + 208;
    w.shq = dw_shift(pl);  // == dw_shift(ph)
    w.shs = dw_shift(ps);
    w.shd = dw_shift(pd);
    load9(dw_floor(pl), w.rl);
    load9(dw_floor(ph), w.rh);
    const u32x2_t s2 = gload<u32x2_a4_t>(dw_floor(ps));  // bytes ps..ps+5 (shift <= 2)
    w.rs[0] = s2[0];
    w.rs[1] = s2[1];
    w.rd = gload<uint32_t>(dw_floor(pd));
  }
  __device__ static void finish(W& w, const uint32_t*) {
    realign8(w.rl, w.shq, w.ql);
    realign8(w.rh, w.shq, w.qh);
    const uint32_t lo = __builtin_amdgcn_alignbyte(w.rs[1], w.rs[0], w.shs);  // scales[0..3] from ps
    const uint32_t hi = w.shs ? (w.rs[1] >> (8 * w.shs)) : w.rs[1];         // bytes ps+4, ps+5
    w.sc[0] = (int8_t)(lo & 0xFF);
    w.sc[1] = (int8_t)((lo >> 8) & 0xFF);
    w.sc[2] = (int8_t)(hi & 0xFF);
    w.sc[3] = (int8_t)((hi >> 8) & 0xFF);
    w.d = half_bits_to_float((w.rd >> (8 * w.shd)) & 0xFFFF);
  }
  __device__ static void qblocks(int u, int& ub0, int& ub1) {
    const int v = u & 3;
    ub0 = 8 * (u >> 2) + 4 * (v >> 1) + (v & 1);
    ub1 = ub0 + 2;
  }
  __device__ static void prep(Act<2>& a) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int s = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) s = dot4(0x01010101u, a.q[4 * j + i], s);
      a.s[j] = s;
    }
  }
  __device__ static float dot(const W& w, const Act<2>& a) {
    int s[4] = {0, 0, 0, 0};
    const int sh = 2 * w.c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = (w.ql[i] & 0x0F0F0F0Fu) | (((w.qh[i] >> sh) & 0x03030303u) << 4);
      const uint32_t hi = ((w.ql[i] >> 4) & 0x0F0F0F0Fu) | (((w.qh[i] >> (sh + 4)) & 0x03030303u) << 4);
      s[i >> 2] = dot4(lo, a.q[i], s[i >> 2]);
      s[2 + (i >> 2)] = dot4(hi, a.q[8 + i], s[2 + (i >> 2)]);
    }
    const float p0 = (float)(w.sc[0] * (s[0] - 32 * a.s[0]) + w.sc[1] * (s[1] - 32 * a.s[1]));
    const float p1 = (float)(w.sc[2] * (s[2] - 32 * a.s[2]) + w.sc[3] * (s[3] - 32 * a.s[3]));
    return w.d * (a.d[0] * p0 + a.d[1] * p1);
  }
};

// IQ3_S: unit u -> super-block u/8, 32-value group ib = u%8. Blocks are 110 bytes: fp16 d,
// qs[64], qh[8], signs[32], scales[4].
template <>
struct Unit<GGML_IQ3_S> {
  static constexpr int VALS = 32, NQ = 1;
  static constexpr int NLD = 5;  // VMEM instructions of load(), at least: the compiler merges q2 and rq[2]
  struct W {
    uint32_t rq[3], rg[2], rd, rh, rsc;
    uint32_t shq, shg, shd, shh, shsc;
    int ib;
    uint32_t v[8];
    float db;
  };
  __device__ static uint32_t sign_mask(int bits4) {
    return ((((uint32_t)bits4 * 0x00204081u) & 0x01010101u) * 0xFFu);
  }
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 3) * QBIQ3_S;
    w.ib = u & 7;
    const uint8_t* pq = b + 2 + 8 * w.ib;   // 8 bytes of qs
    const uint8_t* pg = b + 74 + 4 * w.ib;  // 4 bytes of signs
    const uint8_t* ph = b + 66 + w.ib;      // qh byte
    const uint8_t* psc = b + 106 + w.ib / 2;  // scale byte
    w.shq = dw_shift(pq);
    w.shg = dw_shift(pg);
    w.shd = dw_shift(b);
    w.shh = dw_shift(ph);
    w.shsc = dw_shift(psc);
    const uint32_t* fq = dw_floor(pq);
    const u32x2_t q2 = gload<u32x2_a4_t>(fq);
    w.rq[0] = q2[0];
    w.rq[1] = q2[1];
    w.rq[2] = gload<uint32_t>(fq + 2);
    const u32x2_t g2 = gload<u32x2_a4_t>(dw_floor(pg));
    w.rg[0] = g2[0];
    w.rg[1] = g2[1];
    w.rd = gload<uint32_t>(dw_floor(b));
    w.rh = gload<uint32_t>(dw_floor(ph));
    w.rsc = gload<uint32_t>(dw_floor(psc));
  }
  __device__ static void finish(W& w, const uint32_t* grid) {
    const float d = half_bits_to_float((w.rd >> (8 * w.shd)) & 0xFFFF);
    const int nib = (int)((w.rsc >> (8 * w.shsc + 4 * (w.ib & 1))) & 15);
    w.db = d * (float)(1 + 2 * nib);
    const int qh = (int)((w.rh >> (8 * w.shh)) & 0xFF);
    const uint32_t qs[2] = {__builtin_amdgcn_alignbyte(w.rq[1], w.rq[0], w.shq),
                            __builtin_amdgcn_alignbyte(w.rq[2], w.rq[1], w.shq)};
    const uint32_t sg = __builtin_amdgcn_alignbyte(w.rg[1], w.rg[0], w.shg);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const int sb = (sg >> (8 * l)) & 0xFF;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int k = 2 * l + sub;
        const int idx = ((qs[k >> 2] >> (8 * (k & 3))) & 0xFF) | (((qh >> k) & 1) << 8);
        const uint32_t g = grid[idx];
        const uint32_t m = sign_mask(sub ? (sb >> 4) : (sb & 15));
        w.v[k] = (g ^ m) + (m & 0x01010101u);  // per-byte negate where m = 0xFF (g >= 1: no carry)
      }
    }
  }
  __device__ static void qblocks(int u, int& ub0, int& ub1) { ub0 = ub1 = u; }
  __device__ static void prep(Act<1>&) {}
  __device__ static float dot(const W& w, const Act<1>& a) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = dot4(w.v[i], a.q[i], s);
    return w.db * a.d[0] * (float)s;
  }
};

}  // namespace gemv
}  // namespace ktmi
