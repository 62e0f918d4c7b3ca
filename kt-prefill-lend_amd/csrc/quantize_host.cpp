// Host (CPU) GGUF quantisers: fp32 rows -> Q8_0 / Q4_K / Q6_K / IQ3_S blocks. They build
// expert weights for tests and benchmarks (GGUF checkpoints come from llama.cpp's
// quantisers; any valid encoding exercises the same decode paths). Block layouts are the
// ones decoded in formats.h.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "../../include/ktmi.h"

namespace {

const uint32_t kGrid[512] = {
#include "iq3s_grid.inc"
};

// IEEE fp32 -> fp16 bits, round to nearest even (finite inputs)
uint16_t f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
  uint32_t mant = x & 0x7FFFFFu;
  if (((x >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0));
  if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
  if (exp <= 0) {
    if (exp < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    const int shift = 14 - exp;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)exp << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return (uint16_t)(sign | h);
}

float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1F, mant = h & 0x3FFu;
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else {
      exp = 127 - 15 + 1;
      while (!(mant & 0x400u)) {
        mant <<= 1;
        --exp;
      }
      mant &= 0x3FFu;
      x = sign | (exp << 23) | (mant << 13);
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

void put_h(uint8_t* p, float v) {
  const uint16_t h = f2h(v);
  p[0] = h & 0xFF;
  p[1] = h >> 8;
}

int nearest_int(float v) { return (int)std::lround(v); }

void quant_q8_0(const float* x, uint8_t* b) {
  float amax = 0.f;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
  const float d = amax / 127.f;
  const float dh = h2f(f2h(d));
  const float id = dh > 0.f ? 1.f / dh : 0.f;
  put_h(b, d);
  for (int i = 0; i < 32; ++i) b[2 + i] = (uint8_t)(int8_t)std::clamp(nearest_int(x[i] * id), -127, 127);
}

void quant_q4_k(const float* x, uint8_t* b) {
  float scale[8], mins[8];
  for (int j = 0; j < 8; ++j) {
    float mn = x[32 * j], mx = x[32 * j];
    for (int i = 1; i < 32; ++i) {
      mn = std::min(mn, x[32 * j + i]);
      mx = std::max(mx, x[32 * j + i]);
    }
    if (mn > 0.f) mn = 0.f;
    scale[j] = (mx - mn) / 15.f;
    mins[j] = -mn;
  }
  float ms = 0.f, mm = 0.f;
  for (int j = 0; j < 8; ++j) {
    ms = std::max(ms, scale[j]);
    mm = std::max(mm, mins[j]);
  }
  const float d = h2f(f2h(ms / 63.f)), dmin = h2f(f2h(mm / 63.f));
  int sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = d > 0.f ? std::clamp(nearest_int(scale[j] / d), 0, 63) : 0;
    m[j] = dmin > 0.f ? std::clamp(nearest_int(mins[j] / dmin), 0, 63) : 0;
  }
  memset(b, 0, 144);
  put_h(b, ms / 63.f);
  put_h(b + 2, mm / 63.f);
  uint8_t* s = b + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
  uint8_t* qs = b + 16;
  for (int e = 0; e < 256; ++e) {
    const int j = e / 32;
    const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
    const int q = ds > 0.f ? std::clamp(nearest_int((x[e] + dm) / ds), 0, 15) : 0;
    const int g = e / 64, l = e % 64;
    if (l < 32) qs[32 * g + l] |= (uint8_t)q;
    else qs[32 * g + l - 32] |= (uint8_t)(q << 4);
  }
}

void quant_q6_k(const float* x, uint8_t* b) {
  float scale[16];
  float ms = 0.f;
  for (int g = 0; g < 16; ++g) {
    float amax = 0.f;
    for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * g + i]));
    scale[g] = amax / 31.f;
    ms = std::max(ms, scale[g]);
  }
  const float d = h2f(f2h(ms / 127.f));
  int sc[16];
  for (int g = 0; g < 16; ++g) sc[g] = d > 0.f ? std::clamp(nearest_int(scale[g] / d), -128, 127) : 0;
  memset(b, 0, 210);
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  for (int g = 0; g < 16; ++g) b[192 + g] = (uint8_t)(int8_t)sc[g];
  put_h(b + 208, ms / 127.f);
  for (int e = 0; e < 256; ++e) {
    const int h = e / 128, r = e % 128, c = r / 32, l = r % 32;
    const int g = 8 * h + l / 16 + 2 * c;  // the scale index the decoder uses for e
    const float ds = d * (float)sc[g];
    const int q = ds != 0.f ? std::clamp(nearest_int(x[e] / ds), -32, 31) : 0;
    const int u = q + 32;
    const int li = 64 * h + l + 32 * (c & 1);
    ql[li] |= (uint8_t)(c < 2 ? (u & 15) : ((u & 15) << 4));
    qh[32 * h + l] |= (uint8_t)(((u >> 4) & 3) << (2 * c));
  }
}

struct GridSoA {
  float g[4][512];
  float n2[512];
  GridSoA() {
    for (int i = 0; i < 512; ++i) {
      float s = 0.f;
      for (int k = 0; k < 4; ++k) {
        g[k][i] = (float)((kGrid[i] >> (8 * k)) & 0xFF);
        s += g[k][i] * g[k][i];
      }
      n2[i] = s;
    }
  }
};
const GridSoA& grid_soa() {
  static const GridSoA g;
  return g;
}

// index of the codebook point nearest (L2) to v[4]
int nearest_grid(const float v[4]) {
  const GridSoA& G = grid_soa();
  float best = INFINITY;
  int bi = 0;
  for (int i = 0; i < 512; ++i) {
    const float dist = G.n2[i] - 2.f * (G.g[0][i] * v[0] + G.g[1][i] * v[1] + G.g[2][i] * v[2] + G.g[3][i] * v[3]);
    if (dist < best) {
      best = dist;
      bi = i;
    }
  }
  return bi;
}

void quant_iq3_s(const float* x, uint8_t* b) {
  float s[8];
  float ms = 0.f;
  for (int ib = 0; ib < 8; ++ib) {
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[32 * ib + i]));
    s[ib] = amax / 15.f;
    ms = std::max(ms, s[ib]);
  }
  const float d = h2f(f2h(ms / 31.f));
  memset(b, 0, 110);
  put_h(b, ms / 31.f);
  for (int ib = 0; ib < 8; ++ib) {
    const int nib = d > 0.f ? std::clamp(nearest_int((s[ib] / d - 1.f) / 2.f), 0, 15) : 0;
    b[106 + ib / 2] |= (uint8_t)(nib << (4 * (ib % 2)));
    const float db = d * (float)(1 + 2 * nib);
    for (int l = 0; l < 4; ++l) {
      uint8_t sg = 0;
      for (int sub = 0; sub < 2; ++sub) {
        float v[4];
        for (int k = 0; k < 4; ++k) {
          const float xv = x[32 * ib + 8 * l + 4 * sub + k];
          v[k] = db > 0.f ? std::fabs(xv) / db : 0.f;
          if (xv < 0.f) sg |= (uint8_t)(1u << (4 * sub + k));
        }
        const int idx = nearest_grid(v);
        b[2 + 8 * ib + 2 * l + sub] = (uint8_t)(idx & 0xFF);
        b[66 + ib] |= (uint8_t)(((idx >> 8) & 1) << (2 * l + sub));
      }
      b[74 + 4 * ib + l] = sg;
    }
  }
}

}  // namespace

extern "C" int ktmi_quantize_rows_host(const float* x, int64_t rows, int64_t cols, int ggml_type, void* out,
                                       int threads) {
  int qk, qb;
  void (*fn)(const float*, uint8_t*);
  switch (ggml_type) {
    case 8: qk = 32; qb = 34; fn = quant_q8_0; break;
    case 12: qk = 256; qb = 144; fn = quant_q4_k; break;
    case 14: qk = 256; qb = 210; fn = quant_q6_k; break;
    case 21: qk = 256; qb = 110; fn = quant_iq3_s; break;
    default: return KTMI_ETYPE;
  }
  if (rows < 0 || cols <= 0 || cols % qk || (rows > 0 && (!x || !out))) return KTMI_EINVAL;
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  const int64_t nb = cols / qk;
  const int64_t total = rows * nb;
  threads = (int)std::min<int64_t>(threads, std::max<int64_t>(1, total / 64));
  auto work = [&](int64_t b0, int64_t b1) {
    for (int64_t i = b0; i < b1; ++i) fn(x + i * qk, (uint8_t*)out + i * qb);
  };
  if (threads <= 1) {
    work(0, total);
    return KTMI_OK;
  }
  std::vector<std::thread> pool;
  const int64_t per = (total + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const int64_t b0 = t * per, b1 = std::min(total, b0 + per);
    if (b0 < b1) pool.emplace_back(work, b0, b1);
  }
  for (auto& th : pool) th.join();
  return KTMI_OK;
}
