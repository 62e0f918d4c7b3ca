/* CPU expert path restated in C: TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py
 * times beside the GPU, and a second oracle for the layer output). Never linked into the
 * product.
 *
 * Follows the structure and numerics of kt-kernel's LLAMAFILE MoE forward_many (reference
 * trees/kt-kernel/kt-kernel-95009ea-flash-next-gguf.patch K:2571-2800; the kt-kernel and
 * llama.cpp sources themselves are not in the reference, so the block dot products are
 * restated from the GGUF formats):
 *   1. routes grouped per expert (m_local_num / m_local_pos, K:2645-2680);
 *   2. each token's activation row quantised once to the gate/up vec-dot type: Q8_K
 *      (per 256: fp32 d, int8 q, int16 sums per 16) for the K-quants and IQ3_S, Q8_0 for
 *      Q8_0;
 *   3. gate and up rows per expert as int8 block dot products, row blocks spread over the
 *      threads (many_row_block, K:2287);
 *   4. act_fn(gate) * up in fp32 (x / (1 + expf(-x)), K:2473), re-quantised to the down
 *      vec-dot type;
 *   5. down rows per expert, then the fp32 weighted merge over k in route order
 *      (K:2742-2790).
 * Threads: OpenMP, `threads` of them.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>


#define T_Q8_0 8
#define T_Q4_K 12
#define T_Q6_K 14
#define T_IQ3_S 21

/* the IQ3_S codebook (format data, hash-checked by the tests) */
static const uint32_t ktmi_iq3s_grid_c[512] = {
#include "../kt-prefill-lend_amd/csrc/iq3s_grid.inc"
};

static float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1F, mant = h & 0x3FFu, x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else {
      exp = 127 - 15 + 1;
      while (!(mant & 0x400u)) {
        mant <<= 1;
        --exp;
      }
      x = sign | (exp << 23) | ((mant & 0x3FFu) << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7F800000u | (mant << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}
static uint16_t f2h(float f) { /* round to nearest even, finite inputs */
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t e = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
  uint32_t mant = x & 0x7FFFFFu;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    const int sh = 14 - e;
    uint32_t hm = mant >> sh;
    const uint32_t rem = mant & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (hm & 1))) ++hm;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = ((uint32_t)e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) ++hm;
  return (uint16_t)(sign | hm);
}
static float bf2f(uint16_t b) {
  uint32_t x = (uint32_t)b << 16;
  float f;
  memcpy(&f, &x, 4);
  return f;
}
static int nearest(float v) { return (int)lrintf(v); }

/* ---- activation formats */
typedef struct {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
} q8k_t;
typedef struct {
  uint16_t d;
  int8_t qs[32];
} q8_0_t;

static int is_k(int t) { return t != T_Q8_0; }
static size_t vd_row_bytes(int t, int n) { return is_k(t) ? (size_t)(n / 256) * sizeof(q8k_t) : (size_t)(n / 32) * sizeof(q8_0_t); }
static size_t w_row_bytes(int t, int n) {
  switch (t) {
    case T_Q8_0: return (size_t)(n / 32) * 34;
    case T_Q4_K: return (size_t)(n / 256) * 144;
    case T_Q6_K: return (size_t)(n / 256) * 210;
    default: return (size_t)(n / 256) * 110;
  }
}

static void quant_q8k(const float* x, int n, q8k_t* y) {
  for (int b = 0; b < n / 256; ++b, x += 256) {
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 256; ++j) {
      const float a = fabsf(x[j]);
      if (a > amax) {
        amax = a;
        mx = x[j];
      }
    }
    if (amax == 0.f) {
      memset(&y[b], 0, sizeof(q8k_t));
      continue;
    }
    const float iscale = -127.f / mx;
    for (int j = 0; j < 256; ++j) {
      int v = nearest(iscale * x[j]);
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
static void quant_q8_0(const float* x, int n, q8_0_t* y) {
  for (int b = 0; b < n / 32; ++b, x += 32) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.f, id = d ? 1.f / d : 0.f;
    y[b].d = f2h(d);
    for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t)nearest(x[j] * id);
  }
}
static void quant_vd(int t, const float* x, int n, void* y) {
  if (is_k(t)) quant_q8k(x, n, (q8k_t*)y);
  else quant_q8_0(x, n, (q8_0_t*)y);
}

/* ---- block dot products (weight row . quantised activation row) */
static inline int dot32_i8(const int8_t* a, const int8_t* b) {
  int s = 0;
  for (int i = 0; i < 32; ++i) s += (int)a[i] * (int)b[i];
  return s;
}

static float vdot_q8_0(const uint8_t* w, const q8_0_t* x, int n) {
  float acc = 0.f;
  for (int b = 0; b < n / 32; ++b) {
    const uint8_t* blk = w + 34 * b;
    uint16_t dh;
    memcpy(&dh, blk, 2);
    acc += h2f(dh) * h2f(x[b].d) * (float)dot32_i8((const int8_t*)(blk + 2), x[b].qs);
  }
  return acc;
}

static void q4k_sm(const uint8_t* s, int j, int* sc, int* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

static float vdot_q4_k(const uint8_t* w, const q8k_t* x, int n) {
  float acc = 0.f;
  for (int b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 144 * b;
    uint16_t hd, hm;
    memcpy(&hd, blk, 2);
    memcpy(&hm, blk + 2, 2);
    const uint8_t* qs = blk + 16;
    int8_t q[256];
    for (int g = 0; g < 4; ++g)
      for (int l = 0; l < 32; ++l) {
        q[64 * g + l] = (int8_t)(qs[32 * g + l] & 15);
        q[64 * g + 32 + l] = (int8_t)(qs[32 * g + l] >> 4);
      }
    int sumi = 0, summ = 0;
    for (int j = 0; j < 8; ++j) {
      int sc, m;
      q4k_sm(blk + 4, j, &sc, &m);
      sumi += sc * dot32_i8(q + 32 * j, x[b].qs + 32 * j);
      summ += m * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
    }
    acc += h2f(hd) * x[b].d * (float)sumi - h2f(hm) * x[b].d * (float)summ;
  }
  return acc;
}

static float vdot_q6_k(const uint8_t* w, const q8k_t* x, int n) {
  float acc = 0.f;
  for (int b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 210 * b;
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    uint16_t hd;
    memcpy(&hd, blk + 208, 2);
    int8_t q[256];
    for (int h = 0; h < 2; ++h)
      for (int l = 0; l < 32; ++l) {
        const uint8_t lo0 = ql[64 * h + l], lo1 = ql[64 * h + 32 + l], hb = qh[32 * h + l];
        q[128 * h + l] = (int8_t)(((lo0 & 15) | (((hb >> 0) & 3) << 4)) - 32);
        q[128 * h + 32 + l] = (int8_t)(((lo1 & 15) | (((hb >> 2) & 3) << 4)) - 32);
        q[128 * h + 64 + l] = (int8_t)(((lo0 >> 4) | (((hb >> 4) & 3) << 4)) - 32);
        q[128 * h + 96 + l] = (int8_t)(((lo1 >> 4) | (((hb >> 6) & 3) << 4)) - 32);
      }
    int sumi = 0;
    for (int g = 0; g < 16; ++g) {
      int s = 0;
      for (int i = 0; i < 16; ++i) s += (int)q[16 * g + i] * (int)x[b].qs[16 * g + i];
      sumi += sc[g] * s;
    }
    acc += h2f(hd) * x[b].d * (float)sumi;
  }
  return acc;
}

static float vdot_iq3_s(const uint8_t* w, const q8k_t* x, int n) {
  float acc = 0.f;
  for (int b = 0; b < n / 256; ++b) {
    const uint8_t* blk = w + 110 * b;
    uint16_t hd;
    memcpy(&hd, blk, 2);
    int sum = 0;
    for (int ib = 0; ib < 8; ++ib) {
      const int ls = 2 * ((blk[106 + ib / 2] >> (4 * (ib & 1))) & 15) + 1;
      const int qh = blk[66 + ib];
      int8_t v[32];
      for (int l = 0; l < 4; ++l) {
        const int sg = blk[74 + 4 * ib + l];
        for (int sub = 0; sub < 2; ++sub) {
          const int idx = blk[2 + 8 * ib + 2 * l + sub] | (((qh >> (2 * l + sub)) & 1) << 8);
          const uint32_t g = ktmi_iq3s_grid_c[idx];
          for (int k = 0; k < 4; ++k) {
            const int jj = 4 * sub + k;
            const int gv = (g >> (8 * k)) & 0xFF;
            v[8 * l + jj] = (int8_t)(((sg >> jj) & 1) ? -gv : gv);
          }
        }
      }
      sum += ls * dot32_i8(v, x[b].qs + 32 * ib);
    }
    acc += h2f(hd) * x[b].d * (float)sum;
  }
  return acc;
}

static float vdot(int t, const uint8_t* w, const void* x, int n) {
  switch (t) {
    case T_Q8_0: return vdot_q8_0(w, (const q8_0_t*)x, n);
    case T_Q4_K: return vdot_q4_k(w, (const q8k_t*)x, n);
    case T_Q6_K: return vdot_q6_k(w, (const q8k_t*)x, n);
    default: return vdot_iq3_s(w, (const q8k_t*)x, n);
  }
}

static int row_block(int rows) {
  for (int b = 256; b > 32; b /= 2)
    if (rows % b == 0) return b;
  return 32;
}

/* One MoE layer's routes with slot_ids >= 0: out [T, K] fp32. Returns 0 or -1. */
int cpu_moe_forward(int T, int K, int N, int top_k, int n_slots, const uint16_t* x_bf16, const int32_t* slot_ids,
                    const float* wts, const uint8_t* w13, const uint8_t* w2, int type13, int type2, float* out,
                    int threads) {
  if (threads > 0) omp_set_num_threads(threads);
  const size_t rb13 = w_row_bytes(type13, K), rb2 = w_row_bytes(type2, N);
  const size_t xrb = vd_row_bytes(type13, K), hrb = vd_row_bytes(type2, N);
  int* cnt = (int*)calloc(n_slots + 1, sizeof(int));
  int* pos = (int*)malloc(sizeof(int) * (size_t)T * top_k);
  if (!cnt || !pos) return -1;
  for (int p = 0; p < T * top_k; ++p) {
    const int e = slot_ids[p];
    pos[p] = (e >= 0 && e < n_slots) ? cnt[e]++ : -1;
  }
  int* off = (int*)calloc(n_slots + 1, sizeof(int));
  for (int e = 0; e < n_slots; ++e) off[e + 1] = off[e] + cnt[e];
  const int R = off[n_slots];
  int* tok = (int*)malloc(sizeof(int) * (R > 0 ? R : 1));
  for (int p = 0; p < T * top_k; ++p)
    if (pos[p] >= 0) tok[off[slot_ids[p]] + pos[p]] = p / top_k;

  /* 2. activation rows quantised once per token */
  uint8_t* xq = (uint8_t*)malloc(xrb * (size_t)T);
#pragma omp parallel
  {
    float* f = (float*)malloc(sizeof(float) * K);
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t) {
      for (int c = 0; c < K; ++c) f[c] = bf2f(x_bf16[(size_t)t * K + c]);
      quant_vd(type13, f, K, xq + xrb * t);
    }
    free(f);
  }
  /* 3-4. gate/up per (expert, row block), then act * up */
  float* g = (float*)malloc(sizeof(float) * (size_t)(R > 0 ? R : 1) * N);
  float* u = (float*)malloc(sizeof(float) * (size_t)(R > 0 ? R : 1) * N);
  const int mb = row_block(N), nbn = N / mb;
#pragma omp parallel for schedule(dynamic)
  for (int task = 0; task < n_slots * nbn; ++task) {
    const int e = task / nbn, r0 = (task % nbn) * mb;
    if (cnt[e] == 0) continue;
    const uint8_t* we = w13 + (size_t)e * 2 * N * rb13;
    for (int r = r0; r < r0 + mb; ++r)
      for (int m = 0; m < cnt[e]; ++m) {
        const void* xr = xq + xrb * tok[off[e] + m];
        g[(size_t)(off[e] + m) * N + r] = vdot(type13, we + (size_t)r * rb13, xr, K);
        u[(size_t)(off[e] + m) * N + r] = vdot(type13, we + (size_t)(N + r) * rb13, xr, K);
      }
  }
  uint8_t* hq = (uint8_t*)malloc(hrb * (size_t)(R > 0 ? R : 1));
#pragma omp parallel for schedule(static)
  for (int i = 0; i < R; ++i) {
    float* a = g + (size_t)i * N;
    for (int r = 0; r < N; ++r) a[r] = a[r] / (1.f + expf(-a[r])) * u[(size_t)i * N + r];
    quant_vd(type2, a, N, hq + hrb * i);
  }
  /* 5. down per (expert, row block of K), then the weighted merge */
  float* d = (float*)malloc(sizeof(float) * (size_t)(R > 0 ? R : 1) * K);
  const int kb = row_block(K), nbk = K / kb;
#pragma omp parallel for schedule(dynamic)
  for (int task = 0; task < n_slots * nbk; ++task) {
    const int e = task / nbk, c0 = (task % nbk) * kb;
    if (cnt[e] == 0) continue;
    const uint8_t* we = w2 + (size_t)e * K * rb2;
    for (int c = c0; c < c0 + kb; ++c)
      for (int m = 0; m < cnt[e]; ++m)
        d[(size_t)(off[e] + m) * K + c] = vdot(type2, we + (size_t)c * rb2, hq + hrb * (off[e] + m), N);
  }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    float* o = out + (size_t)t * K;
    for (int c = 0; c < K; ++c) o[c] = 0.f;
    for (int k = 0; k < top_k; ++k) {
      const int p = t * top_k + k;
      if (pos[p] < 0) continue;
      const float* dr = d + (size_t)(off[slot_ids[p]] + pos[p]) * K;
      const float wk = wts[p];
      for (int c = 0; c < K; ++c) o[c] += dr[c] * wk;
    }
  }
  free(cnt);
  free(pos);
  free(off);
  free(tok);
  free(xq);
  free(g);
  free(u);
  free(hq);
  free(d);
  return 0;
}

int cpu_moe_max_threads(void) { return omp_get_max_threads(); }
