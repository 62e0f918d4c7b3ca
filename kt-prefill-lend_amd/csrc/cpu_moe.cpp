// CPU expert engine: the cold routes of a MoE layer on the host cores, with the numerics of
// kt-kernel's LLAMAFILE MoE forward_many (reference trees/kt-kernel/
// kt-kernel-95009ea-flash-next-gguf.patch K:2571-2800):
//   1. routes grouped per expert in route order (m_local_num / m_local_pos, K:2645-2680);
//   2. each token's bf16 activation row quantised once to the gate/up vec-dot type: Q8_K
//      (per 256 values: fp32 d = 1/iscale with iscale = -127/max, the value of largest
//      magnitude; int8 codes rounded to nearest even; int16 sums per 16) for the K-quants
//      and IQ3_S, Q8_0 (fp16 d = amax/127) for Q8_0;
//   3. gate and up rows per expert as int8 block dot products, over (expert, row block)
//      tasks spread on a thread pool, each task ending with silu(gate) * up of its rows in
//      fp32 (x / (1 + expf(-x)) * up, K:2473);
//   4. h re-quantised to the down vec-dot type;
//   5. down rows per expert, then per token the fp32 sum over k in route order of
//      y * w, rounded once to bf16.
// Within a block, the integer dot products are exact (AVX-512 VNNI `vpdpbusd` when the host
// has it, a scalar loop otherwise) and the per-block fp32 arithmetic has one fixed order,
// so both kernels give bit-identical results. Built without floating-point contraction.
#include "cpu_moe.h"

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <immintrin.h>
#include <sched.h>

namespace ktmi_cpu {
namespace {

constexpr int T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_IQ3_S = 21;

const uint32_t kGrid[512] = {
#include "iq3s_grid.inc"
};

float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FFu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int sh = 0;
      while (!(m & 0x400u)) {
        m <<= 1;
        ++sh;
      }
      bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t f2h(float f) {  // round to nearest even, finite non-negative scales
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t e = (int32_t)((x >> 23) & 0xFF) - 112;
  uint32_t m = x & 0x7FFFFFu;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const int sh = 14 - e;
    uint32_t hm = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (hm & 1))) ++hm;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) ++hm;
  return (uint16_t)(sign | hm);
}

inline float bf2f(uint16_t b) {
  const uint32_t x = (uint32_t)b << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}

inline uint16_t f2bf(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return (uint16_t)((x >> 16) | 0x40);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1)) >> 16);
}

// ---- activation blocks
struct Q8K {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
};
struct Q80 {
  uint16_t d;
  int8_t qs[32];
};
static_assert(sizeof(Q8K) == 292 && sizeof(Q80) == 34, "block sizes");

bool is_k(int t) { return t != T_Q8_0; }
size_t vd_row_bytes(int t, int64_t n) { return is_k(t) ? (size_t)(n / 256) * sizeof(Q8K) : (size_t)(n / 32) * sizeof(Q80); }
size_t w_row_bytes(int t, int64_t n) {
  switch (t) {
    case T_Q8_0: return (size_t)(n / 32) * 34;
    case T_Q4_K: return (size_t)(n / 256) * 144;
    case T_Q6_K: return (size_t)(n / 256) * 210;
    default: return (size_t)(n / 256) * 110;
  }
}
int64_t block_of(int t) { return t == T_Q8_0 ? 32 : 256; }

void quant_q8k(const float* x, int64_t n, Q8K* y) {
  for (int64_t b = 0; b < n / 256; ++b, x += 256) {
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 256; ++j) {
      const float a = std::fabs(x[j]);
      if (a > amax) {
        amax = a;
        mx = x[j];
      }
    }
    if (amax == 0.f) {
      memset(&y[b], 0, sizeof(Q8K));
      continue;
    }
    const float iscale = -127.f / mx;
    for (int j = 0; j < 256; ++j) {
      const long v = std::lrint(iscale * x[j]);
      y[b].qs[j] = (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
    }
    for (int g = 0; g < 16; ++g) {
      int s = 0;
      for (int j = 0; j < 16; ++j) s += y[b].qs[16 * g + j];
      y[b].bsums[g] = (int16_t)s;
    }
    y[b].d = 1.f / iscale;
  }
}

void quant_q80(const float* x, int64_t n, Q80* y) {
  for (int64_t b = 0; b < n / 32; ++b, x += 32) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.f, id = d != 0.f ? 1.f / d : 0.f;
    y[b].d = f2h(d);
    for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t)std::lrint(x[j] * id);
  }
}

void quant_vd(int t, const float* x, int64_t n, uint8_t* y) {
  if (is_k(t)) quant_q8k(x, n, (Q8K*)y);
  else quant_q80(x, n, (Q80*)y);
}

void q4k_scale_min(const uint8_t* s, int j, int& sc, int& m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// ---- scalar block dot products (weight row . quantised activation row)
float dot_q80_scalar(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q80* x = (const Q80*)xv;
  float acc = 0.f;
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = w + 34 * b;
    uint16_t dh;
    memcpy(&dh, blk, 2);
    const int8_t* q = (const int8_t*)(blk + 2);
    int s = 0;
    for (int i = 0; i < 32; ++i) s += (int)q[i] * (int)x[b].qs[i];
    acc += h2f(dh) * h2f(x[b].d) * (float)s;
  }
  return acc;
}

float dot_q4k_scalar(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 144 * b;
    uint16_t hd, hm;
    memcpy(&hd, blk, 2);
    memcpy(&hm, blk + 2, 2);
    int sumi = 0, summ = 0;
    for (int j = 0; j < 8; ++j) {
      int sc, m;
      q4k_scale_min(blk + 4, j, sc, m);
      const uint8_t* qs = blk + 16 + 32 * (j / 2);
      const int8_t* xq = x[b].qs + 32 * j;
      int s = 0;
      for (int l = 0; l < 32; ++l) s += (int)((j & 1) ? (qs[l] >> 4) : (qs[l] & 15)) * (int)xq[l];
      sumi += sc * s;
      summ += m * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
    }
    acc += h2f(hd) * x[b].d * (float)sumi - h2f(hm) * x[b].d * (float)summ;
  }
  return acc;
}

float dot_q6k_scalar(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 210 * b;
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    uint16_t hd;
    memcpy(&hd, blk + 208, 2);
    int sumi = 0;
    for (int g = 0; g < 16; ++g) {  // 16 values: half h, run c, 16-group within the run
      const int h = g / 8, c = (g / 2) % 4, l0 = 16 * (g % 2);
      int s = 0;
      for (int l = l0; l < l0 + 16; ++l) {
        const uint8_t lo = ql[64 * h + l + 32 * (c & 1)];
        const int nib = c < 2 ? (lo & 15) : (lo >> 4);
        const int hi = (qh[32 * h + l] >> (2 * c)) & 3;
        s += ((nib | (hi << 4)) - 32) * (int)x[b].qs[16 * g + (l - l0)];
      }
      sumi += sc[g] * s;
    }
    acc += h2f(hd) * x[b].d * (float)sumi;
  }
  return acc;
}

float dot_iq3s_scalar(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 110 * b;
    uint16_t hd;
    memcpy(&hd, blk, 2);
    int sum = 0;
    for (int ib = 0; ib < 8; ++ib) {
      const int ls = 2 * ((blk[106 + ib / 2] >> (4 * (ib & 1))) & 15) + 1;
      const int qh = blk[66 + ib];
      uint32_t sg;
      memcpy(&sg, blk + 74 + 4 * ib, 4);
      int s = 0;
      for (int k = 0; k < 8; ++k) {
        const uint32_t g = kGrid[blk[2 + 8 * ib + k] | (((qh >> k) & 1) << 8)];
        for (int j = 0; j < 4; ++j) {
          const int pos = 4 * k + j;
          const int gv = (int)((g >> (8 * j)) & 0xFF);
          s += (((sg >> pos) & 1) ? -gv : gv) * (int)x[b].qs[32 * ib + pos];
        }
      }
      sum += ls * s;
    }
    acc += h2f(hd) * x[b].d * (float)sum;
  }
  return acc;
}

// ---- AVX-512 VNNI block dot products (same integers, same fp32 order)
#define KT_VNNI __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,f16c")))

// fp16 -> fp32 with the F16C instruction (exact, as h2f)
KT_VNNI inline float h2f_hw(uint16_t h) { return _cvtsh_ss(h); }

KT_VNNI inline int hsum8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
}

KT_VNNI float dot_q80_vnni(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q80* x = (const Q80*)xv;
  float acc = 0.f;
  for (int64_t b = 0; b < n / 32; ++b) {
    const uint8_t* blk = w + 34 * b;
    uint16_t dh;
    memcpy(&dh, blk, 2);
    const __m256i q = _mm256_loadu_si256((const __m256i*)(blk + 2));
    const __m256i xq = _mm256_loadu_si256((const __m256i*)x[b].qs);
    // |q| (unsigned) times x with q's sign: exact for |x| <= 127 (the Q8_0 activation codes)
    const __m256i d = _mm256_dpbusd_epi32(_mm256_setzero_si256(), _mm256_abs_epi8(q), _mm256_sign_epi8(xq, q));
    acc += h2f_hw(dh) * h2f_hw(x[b].d) * (float)hsum8(d);
  }
  return acc;
}

KT_VNNI float dot_q4k_vnni(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 144 * b;
    uint16_t hd, hm;
    memcpy(&hd, blk, 2);
    memcpy(&hm, blk + 2, 2);
    __m256i sv = _mm256_setzero_si256();
    // the eight 6-bit scales and mins of q4k_scale_min, four bytes at a time: sub-blocks
    // 0-3 are the low 6 bits of bytes 0-3 (scales) and 4-7 (mins); sub-blocks 4-7 take their
    // low 4 bits from bytes 8-11 and their high 2 bits from bits 6-7 of bytes 0-3 / 4-7
    uint32_t w1, w2, w3;
    memcpy(&w1, blk + 4, 4);
    memcpy(&w2, blk + 8, 4);
    memcpy(&w3, blk + 12, 4);
    const uint32_t scl = w1 & 0x3F3F3F3Fu, mnl = w2 & 0x3F3F3F3Fu;
    const uint32_t sch = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    const uint32_t mnh = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
    for (int g = 0; g < 4; ++g) {
      const uint32_t scw = g < 2 ? scl : sch;
      const int sh = 16 * (g & 1);
      const int sc0 = (int)((scw >> sh) & 0xFF), sc1 = (int)((scw >> (sh + 8)) & 0xFF);
      const __m256i q = _mm256_loadu_si256((const __m256i*)(blk + 16 + 32 * g));
      const __m256i lo = _mm256_and_si256(q, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
      const __m256i dl = _mm256_dpbusd_epi32(_mm256_setzero_si256(), lo,
                                             _mm256_loadu_si256((const __m256i*)(x[b].qs + 64 * g)));
      const __m256i dh = _mm256_dpbusd_epi32(_mm256_setzero_si256(), hi,
                                             _mm256_loadu_si256((const __m256i*)(x[b].qs + 64 * g + 32)));
      sv = _mm256_add_epi32(sv, _mm256_mullo_epi32(dl, _mm256_set1_epi32(sc0)));
      sv = _mm256_add_epi32(sv, _mm256_mullo_epi32(dh, _mm256_set1_epi32(sc1)));
    }
    // sum over sub-blocks j of m_j * (bsums[2j] + bsums[2j+1]): each min byte doubled to two
    // int16 lanes against the 16 int16 bsums (exact in int32)
    const __m128i mb = _mm_cvtsi64_si128((long long)(((uint64_t)mnh << 32) | mnl));
    const __m256i mv = _mm256_cvtepu8_epi16(_mm_unpacklo_epi8(mb, mb));
    const int summ = hsum8(_mm256_madd_epi16(_mm256_loadu_si256((const __m256i*)x[b].bsums), mv));
    const int sumi = hsum8(sv);
    acc += h2f_hw(hd) * x[b].d * (float)sumi - h2f_hw(hm) * x[b].d * (float)summ;
  }
  return acc;
}

KT_VNNI float dot_q6k_vnni(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(3);
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 210 * b;
    const int8_t* sc = (const int8_t*)(blk + 192);
    uint16_t hd;
    memcpy(&hd, blk + 208, 2);
    __m256i sv = _mm256_setzero_si256();
    for (int h = 0; h < 2; ++h) {
      const __m256i l0 = _mm256_loadu_si256((const __m256i*)(blk + 64 * h));
      const __m256i l1 = _mm256_loadu_si256((const __m256i*)(blk + 64 * h + 32));
      const __m256i qh = _mm256_loadu_si256((const __m256i*)(blk + 128 + 32 * h));
      // unsigned 6-bit codes of the 4 runs (the -32 offset is applied through the sums)
      __m256i q[4];
      q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4));
      q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                             _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4));
      q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                             _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4));
      q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                             _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4));
      for (int c = 0; c < 4; ++c) {
        const int g = 8 * h + 2 * c;  // the run's two 16-value groups
        const __m256i d = _mm256_dpbusd_epi32(_mm256_setzero_si256(), q[c],
                                              _mm256_loadu_si256((const __m256i*)(x[b].qs + 128 * h + 32 * c)));
        sv = _mm256_add_epi32(sv, _mm256_mullo_epi32(d, _mm256_setr_epi32(sc[g], sc[g], sc[g], sc[g], sc[g + 1],
                                                                          sc[g + 1], sc[g + 1], sc[g + 1])));
      }
    }
    int corr = 0;
    for (int g = 0; g < 16; ++g) corr += sc[g] * x[b].bsums[g];
    const int sumi = hsum8(sv) - 32 * corr;
    acc += h2f_hw(hd) * x[b].d * (float)sumi;
  }
  return acc;
}

KT_VNNI float dot_iq3s_vnni(const uint8_t* w, const uint8_t* xv, int64_t n) {
  const Q8K* x = (const Q8K*)xv;
  const __m256i grid_bias = _mm256_setzero_si256();
  float acc = 0.f;
  for (int64_t b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 110 * b;
    uint16_t hd;
    memcpy(&hd, blk, 2);
    __m256i sv = _mm256_setzero_si256();
    for (int ib = 0; ib < 8; ++ib) {
      const int ls = 2 * ((blk[106 + ib / 2] >> (4 * (ib & 1))) & 15) + 1;
      const int qh = blk[66 + ib];
      alignas(32) int32_t idx[8];
      for (int k = 0; k < 8; ++k) idx[k] = blk[2 + 8 * ib + k] | (((qh >> k) & 1) << 8);
      const __m256i g = _mm256_i32gather_epi32((const int*)kGrid, _mm256_load_si256((const __m256i*)idx), 4);
      uint32_t sg;
      memcpy(&sg, blk + 74 + 4 * ib, 4);
      const __m256i xq = _mm256_loadu_si256((const __m256i*)(x[b].qs + 32 * ib));
      // the weights' signs moved onto the activation codes (|code| <= 127, so negation is exact)
      const __m256i xs = _mm256_mask_sub_epi8(xq, (__mmask32)sg, grid_bias, xq);
      const __m256i d = _mm256_dpbusd_epi32(_mm256_setzero_si256(), g, xs);
      sv = _mm256_add_epi32(sv, _mm256_mullo_epi32(d, _mm256_set1_epi32(ls)));
    }
    acc += h2f_hw(hd) * x[b].d * (float)hsum8(sv);
  }
  return acc;
}

// Q8_K with AVX-512: the codes, sums and scale of quant_q8k (the first value of largest
// magnitude sets iscale = -127 / value; iscale * x rounded to nearest even by the current
// mode, as lrint, then clamped; |iscale * x| <= 127, so the int32 conversion never overflows)
KT_VNNI void quant_q8k_avx512(const float* x, int64_t n, Q8K* y) {
  const __m512i lo = _mm512_set1_epi32(-128), hi = _mm512_set1_epi32(127);
  for (int64_t b = 0; b < n / 256; ++b, x += 256) {
    __m512 vm = _mm512_setzero_ps();
    for (int c = 0; c < 16; ++c) vm = _mm512_max_ps(vm, _mm512_abs_ps(_mm512_loadu_ps(x + 16 * c)));
    const float amax = _mm512_reduce_max_ps(vm);
    if (amax == 0.f) {
      memset(&y[b], 0, sizeof(Q8K));
      continue;
    }
    int j = 0;
    for (int c = 0; c < 16; ++c) {
      const __mmask16 k = _mm512_cmp_ps_mask(_mm512_abs_ps(_mm512_loadu_ps(x + 16 * c)),
                                             _mm512_set1_ps(amax), _CMP_EQ_OQ);
      if (k) {
        j = 16 * c + __builtin_ctz((unsigned)k);
        break;
      }
    }
    const float iscale = -127.f / x[j];
    const __m512 vs = _mm512_set1_ps(iscale);
    for (int c = 0; c < 16; ++c) {
      __m512i v = _mm512_cvtps_epi32(_mm512_mul_ps(vs, _mm512_loadu_ps(x + 16 * c)));
      v = _mm512_min_epi32(_mm512_max_epi32(v, lo), hi);
      _mm_storeu_si128((__m128i*)(y[b].qs + 16 * c), _mm512_cvtepi32_epi8(v));
      y[b].bsums[c] = (int16_t)_mm512_reduce_add_epi32(v);
    }
    y[b].d = 1.f / iscale;
  }
}

using DotFn = float (*)(const uint8_t*, const uint8_t*, int64_t);

// the host has AVX-512 VNNI and KTMI_CPU_ISA does not ask for the portable kernels
bool use_vnni() {
  static const bool hw = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                         __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
  const char* want = getenv("KTMI_CPU_ISA");
  return hw && !(want && strcmp(want, "scalar") == 0);
}

DotFn dot_for(int t, bool v) {
  switch (t) {
    case T_Q8_0: return v ? dot_q80_vnni : dot_q80_scalar;
    case T_Q4_K: return v ? dot_q4k_vnni : dot_q4k_scalar;
    case T_Q6_K: return v ? dot_q6k_vnni : dot_q6k_scalar;
    case T_IQ3_S: return v ? dot_iq3s_vnni : dot_iq3s_scalar;
    default: return nullptr;
  }
}

// ---- a small persistent thread pool: run(n, fn) calls fn(i) for i in [0, n) on the
// workers and the calling thread, dynamic order, and returns when all are done. Workers spin
// on the job counter for a while after each job (a decode layer runs six short phases back
// to back) before they sleep on the condition variable.
class Pool {
 public:
  explicit Pool(int threads) : nw_(threads > 1 ? threads - 1 : 0) {
    for (int i = 0; i < nw_; ++i) th_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(m_);
      stop_.store(true);
      gen_.fetch_add(1);
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  int size() const { return nw_ + 1; }
  void run(int64_t n, const std::function<void(int64_t)>& fn) {
    if (n <= 0) return;
    if (nw_ == 0 || n == 1) {
      for (int64_t i = 0; i < n; ++i) fn(i);
      return;
    }
    fn_ = &fn;
    n_ = n;
    next_.store(0, std::memory_order_relaxed);
    left_.store(nw_, std::memory_order_relaxed);
    {
      std::lock_guard<std::mutex> g(m_);
      gen_.fetch_add(1, std::memory_order_release);
    }
    if (sleepers_.load() > 0) cv_.notify_all();
    work();
    while (left_.load(std::memory_order_acquire) != 0) _mm_pause();
    fn_ = nullptr;
  }

 private:
  void work() {
    for (int64_t i; (i = next_.fetch_add(1, std::memory_order_relaxed)) < n_;) (*fn_)(i);
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      // spin up to 50 microseconds, then sleep
      bool got = false;
      const auto t0 = std::chrono::steady_clock::now();
      for (int i = 0;; ++i) {
        if (gen_.load(std::memory_order_acquire) != seen) {
          got = true;
          break;
        }
        _mm_pause();
        if ((i & 63) == 63 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(50)) break;
      }
      if (!got) {
        std::unique_lock<std::mutex> g(m_);
        sleepers_.fetch_add(1);
        cv_.wait(g, [&] { return gen_.load() != seen; });
        sleepers_.fetch_sub(1);
      }
      seen = gen_.load(std::memory_order_acquire);
      if (stop_.load()) return;
      work();
      left_.fetch_sub(1, std::memory_order_release);
    }
  }
  int nw_;
  std::vector<std::thread> th_;
  std::mutex m_;
  std::condition_variable cv_;
  const std::function<void(int64_t)>* fn_ = nullptr;
  std::atomic<int64_t> next_{0};
  int64_t n_ = 0;
  std::atomic<int> left_{0}, sleepers_{0};
  std::atomic<uint64_t> gen_{0};
  std::atomic<bool> stop_{false};
};

// rows per task: the widest of 256 .. 16 dividing `rows` that still gives every thread
// about four tasks over the active experts (small windows get narrow tasks)
int64_t row_block(int64_t rows, int64_t experts, int threads) {
  int64_t best = 16;
  for (int64_t b = 256; b >= 16; b /= 2) {
    if (rows % b) continue;
    best = b;
    if (experts * (rows / b) >= 4 * threads) break;
  }
  return rows % best ? rows : best;
}

// CPUs in this process's affinity mask (what a container or job scheduler grants), or the
// hardware's count where the mask cannot be read
int usable_cpus() {
  cpu_set_t set;
  CPU_ZERO(&set);
  if (sched_getaffinity(0, sizeof set, &set) == 0) {
    const int n = CPU_COUNT(&set);
    if (n > 0) return n;
  }
  return (int)std::max(1u, std::thread::hardware_concurrency());
}

}  // namespace

struct Engine {
  int64_t K, N, E;
  int t13, t2;
  bool vnni;
  const uint8_t *gate, *up, *down;
  size_t rb13, rb2, xrb, hrb;
  DotFn dot13, dot2;
  const char* isa;
  Pool pool;
  // scratch, grown as needed
  std::vector<int64_t> cnt, off, pos;
  std::vector<int32_t> tok;
  std::vector<uint8_t> xq, hq;
  std::vector<float> g, u, y;
  Engine(int threads) : pool(threads) {}
};

Engine* engine_create(int64_t hidden, int64_t inter, int64_t n_experts, int type13, int type2, const uint8_t* gate,
                      const uint8_t* up, const uint8_t* down, int threads, const char** err) {
  auto fail = [&](const char* m) -> Engine* {
    if (err) *err = m;
    return nullptr;
  };
  const bool vnni = use_vnni();
  if (!dot_for(type13, vnni) || !dot_for(type2, vnni)) return fail("ggml type has no CPU kernel (8, 12, 14, 21)");
  if (hidden <= 0 || inter <= 0 || n_experts <= 0) return fail("non-positive size");
  if (hidden % block_of(type13) || inter % block_of(type2) || hidden % 256 || inter % 32)
    return fail("hidden / intermediate are not whole blocks of the weight and activation types");
  if (!gate || !up || !down) return fail("null bank pointer");
  // default: the CPUs this process may run on (its affinity mask), one of them left to the
  // thread that drives the GPU
  if (threads <= 0) threads = std::max(1, usable_cpus() - 1);
  Engine* e = new Engine(threads);
  e->K = hidden;
  e->N = inter;
  e->E = n_experts;
  e->t13 = type13;
  e->t2 = type2;
  e->gate = gate;
  e->up = up;
  e->down = down;
  e->rb13 = w_row_bytes(type13, hidden);
  e->rb2 = w_row_bytes(type2, inter);
  e->xrb = vd_row_bytes(type13, hidden);
  e->hrb = vd_row_bytes(type2, inter);
  e->dot13 = dot_for(type13, vnni);
  e->dot2 = dot_for(type2, vnni);
  e->isa = vnni ? "avx512-vnni" : "scalar";
  e->vnni = vnni;
  return e;
}

void engine_destroy(Engine* e) { delete e; }

namespace {
// the activation quantiser of the engine's ISA (identical codes either way)
void quant(const Engine* e, int t, const float* x, int64_t n, uint8_t* y) {
  if (e->vnni && is_k(t)) quant_q8k_avx512(x, n, (Q8K*)y);
  else quant_vd(t, x, n, y);
}
}  // namespace

int engine_threads(const Engine* e) { return e->pool.size(); }

const char* engine_isa(const Engine* e) { return e->isa; }

int engine_forward(Engine* e, int64_t T, int64_t top_k, const int32_t* ids, const float* w, const uint16_t* x,
                   uint16_t* out) {
  const int64_t K = e->K, N = e->N, E = e->E, P = T * top_k;
  try {
    // 1. routes grouped per expert, route order inside an expert
    e->cnt.assign(E, 0);
    e->pos.resize(P > 0 ? P : 1);
    for (int64_t p = 0; p < P; ++p) {
      const int32_t ex = ids[p];
      e->pos[p] = (ex >= 0 && ex < E) ? e->cnt[ex]++ : -1;
    }
    e->off.assign(E + 1, 0);
    for (int64_t i = 0; i < E; ++i) e->off[i + 1] = e->off[i] + e->cnt[i];
    const int64_t R = e->off[E];
    e->tok.resize(R > 0 ? R : 1);
    std::vector<int32_t> active;
    for (int64_t p = 0; p < P; ++p)
      if (e->pos[p] >= 0) e->tok[e->off[ids[p]] + e->pos[p]] = (int32_t)(p / top_k);
    for (int64_t i = 0; i < E; ++i)
      if (e->cnt[i]) active.push_back((int32_t)i);
    if (R == 0) {
      e->pool.run(T, [&](int64_t t) { std::fill(out + t * K, out + (t + 1) * K, (uint16_t)0); });
      return 0;
    }
    // 2. activation rows, once per token that has a route here
    e->xq.resize(e->xrb * (size_t)T);
    e->pool.run(T, [&](int64_t t) {
      thread_local std::vector<float> f;
      f.resize(K);
      for (int64_t c = 0; c < K; ++c) f[c] = bf2f(x[t * K + c]);
      quant(e, e->t13, f.data(), K, e->xq.data() + e->xrb * t);
    });
    // 3. gate and up per (active expert, row block), and silu(gate) * up of those rows (in g)
    e->g.resize((size_t)R * N);
    e->u.resize((size_t)R * N);
    const int64_t mb = row_block(N, (int64_t)active.size(), e->pool.size()), nbn = N / mb;
    e->pool.run((int64_t)active.size() * nbn, [&](int64_t task) {
      const int64_t ex = active[task / nbn], r0 = (task % nbn) * mb;
      const uint8_t* wg = e->gate + (size_t)ex * N * e->rb13;
      const uint8_t* wu = e->up + (size_t)ex * N * e->rb13;
      for (int64_t r = r0; r < r0 + mb; ++r)
        for (int64_t m = 0; m < e->cnt[ex]; ++m) {
          const int64_t i = e->off[ex] + m;
          const uint8_t* xr = e->xq.data() + e->xrb * e->tok[i];
          e->g[(size_t)i * N + r] = e->dot13(wg + (size_t)r * e->rb13, xr, K);
          e->u[(size_t)i * N + r] = e->dot13(wu + (size_t)r * e->rb13, xr, K);
        }
      for (int64_t m = 0; m < e->cnt[ex]; ++m) {
        float* a = e->g.data() + (size_t)(e->off[ex] + m) * N;
        const float* b = e->u.data() + (size_t)(e->off[ex] + m) * N;
        for (int64_t r = r0; r < r0 + mb; ++r) a[r] = a[r] / (1.f + std::exp(-a[r])) * b[r];
      }
    });
    // 4. h quantised for the down projection
    e->hq.resize(e->hrb * (size_t)R);
    e->pool.run(R, [&](int64_t i) { quant(e, e->t2, e->g.data() + (size_t)i * N, N, e->hq.data() + e->hrb * i); });
    // 5. down per (active expert, row block of hidden), then the merge in route order
    e->y.resize((size_t)R * K);
    const int64_t kb = row_block(K, (int64_t)active.size(), e->pool.size()), nbk = K / kb;
    e->pool.run((int64_t)active.size() * nbk, [&](int64_t task) {
      const int64_t ex = active[task / nbk], c0 = (task % nbk) * kb;
      const uint8_t* wd = e->down + (size_t)ex * K * e->rb2;
      for (int64_t c = c0; c < c0 + kb; ++c)
        for (int64_t m = 0; m < e->cnt[ex]; ++m) {
          const int64_t i = e->off[ex] + m;
          e->y[(size_t)i * K + c] = e->dot2(wd + (size_t)c * e->rb2, e->hq.data() + e->hrb * i, N);
        }
    });
    e->pool.run(T, [&](int64_t t) {
      thread_local std::vector<float> o;
      o.assign(K, 0.f);
      for (int64_t k = 0; k < top_k; ++k) {
        const int64_t p = t * top_k + k;
        if (e->pos[p] < 0) continue;
        const float* yr = e->y.data() + (size_t)(e->off[ids[p]] + e->pos[p]) * K;
        const float wk = w[p];
        for (int64_t c = 0; c < K; ++c) o[c] += yr[c] * wk;
      }
      for (int64_t c = 0; c < K; ++c) out[t * K + c] = f2bf(o[c]);
    });
  } catch (...) {
    return -1;
  }
  return 0;
}

}  // namespace ktmi_cpu
