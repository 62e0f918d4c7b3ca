// Decode-window MoE GEMV over raw GGUF blocks with int8 activations (wave64).
//
// Contract of kt_moe_a8_vec_multi (hot/kt_gguf_moe_multi/kt_gguf_moe_multi.cu:653-935,
// kernel :75-217): Y[p, r] = row r of expert ids[p] dotted with q8_1(X[p / top_k]) as
// sums of int8 dot products per block scaled by the block scales; ids[p] < 0 gives a
// zero row. Window mode: the first route of an expert computes every route of that
// expert, so its weights stream from HBM once per call; per-route mode: each route on
// its own. The integer sums equal the reference's vec_dot sums (vecdotq.cuh :969-983
// Q8_0, :1326-1367 Q4_K, :1625-1648 Q6_K, :1875-1899 IQ3_S); only the fp32 order of the
// per-block scale products and of the cross-lane reduction differs.
//
// Work split (MI355X-first, not the reference's warp-32 split): a "unit" is the weight
// span one lane decodes per step -- 64 values for Q4_K/Q6_K (32 bytes of packed nibbles
// shared by two sub-blocks), 32 values for Q8_0/IQ3_S. LPR lanes (a power of two <= 64)
// cover one row's units, so a wave64 reads 64/LPR consecutive rows per pass: a contiguous
// byte range of the slot tensor. Each wave runs RITER passes with all their loads issued
// before any dot product, 4 waves per workgroup. Up to 4 routes (members) share every
// weight unit loaded; more members loop in chunks of 4.
#include "formats.h"
#include "kernels.h"

namespace ktmi {

namespace {

constexpr int RITER = 4;
constexpr int WAVES = 4;

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

// ---- per-type weight units

template <int TYPE>
struct Unit;

// Q8_0: unit = block u (32 values, 34 bytes)
template <>
struct Unit<GGML_Q8_0> {
  static constexpr int VALS = 32, NQ = 1;
  struct W { uint32_t q[8]; float d; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)u * QB8_0;
    w.d = half_bits_to_float(ld_u16(b));
    ld16_a2(b + 2, w.q);
    ld16_a2(b + 18, w.q + 4);
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
// and 2g+1 (high nibbles of the same bytes)
template <>
struct Unit<GGML_Q4_K> {
  static constexpr int VALS = 64, NQ = 2;
  struct W { uint32_t q[8]; float d, dmin; int sc0, m0, sc1, m1; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 2) * QB4_K;
    const int g = u & 3;
    const u32x4_t h0 = gload<u32x4_t>(b);  // d, dmin, scales[12]
    const u32x4_t v0 = gload<u32x4_t>(b + 16 + 32 * g);
    const u32x4_t v1 = gload<u32x4_t>(b + 32 + 32 * g);
    w.d = half_bits_to_float(h0[0] & 0xFFFF);
    w.dmin = half_bits_to_float(h0[0] >> 16);
    uint8_t sc[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) sc[i] = (h0[1 + i / 4] >> (8 * (i % 4))) & 0xFF;
    q4k_scale_min(sc, 2 * g, w.sc0, w.m0);
    q4k_scale_min(sc, 2 * g + 1, w.sc1, w.m1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w.q[i] = v0[i];
      w.q[4 + i] = v1[i];
    }
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
template <>
struct Unit<GGML_Q6_K> {
  static constexpr int VALS = 64, NQ = 2;
  struct W { uint32_t ql[8], qh[8]; float d; int sc[4]; int c; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t*, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 2) * QB6_K;
    const int v = u & 3, h = v >> 1, c = v & 1;
    ld16_a2(b + 64 * h + 32 * c, w.ql);
    ld16_a2(b + 64 * h + 32 * c + 16, w.ql + 4);
    ld16_a2(b + 128 + 32 * h, w.qh);
    ld16_a2(b + 128 + 32 * h + 16, w.qh + 4);
    w.d = half_bits_to_float(ld_u16(b + 208));
    const uint8_t* s = b + 192 + 8 * h + 2 * c;
    w.sc[0] = (int8_t)gload<uint8_t>(s);
    w.sc[1] = (int8_t)gload<uint8_t>(s + 1);
    w.sc[2] = (int8_t)gload<uint8_t>(s + 4);
    w.sc[3] = (int8_t)gload<uint8_t>(s + 5);
    w.c = c;
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

// IQ3_S: unit u -> super-block u/8, 32-value group ib = u%8
template <>
struct Unit<GGML_IQ3_S> {
  static constexpr int VALS = 32, NQ = 1;
  struct W { uint32_t v[8]; float db; };
  __device__ static uint32_t sign_mask(int bits4) {
    return ((((uint32_t)bits4 * 0x00204081u) & 0x01010101u) * 0xFFu);
  }
  __device__ static void load(const uint8_t* row, int u, const uint32_t* grid, W& w) {
    const uint8_t* b = row + (int64_t)(u >> 3) * QBIQ3_S;
    const int ib = u & 7;
    const float d = half_bits_to_float(ld_u16(b));
    const int nib = (gload<uint8_t>(b + 106 + ib / 2) >> (4 * (ib & 1))) & 15;
    w.db = d * (float)(1 + 2 * nib);
    const int qh = gload<uint8_t>(b + 66 + ib);
    uint32_t qs[2], sg;
    qs[0] = ld_u32_a2(b + 2 + 8 * ib);
    qs[1] = ld_u32_a2(b + 6 + 8 * ib);
    sg = ld_u32_a2(b + 74 + 4 * ib);
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

template <typename OutT>
__device__ __forceinline__ OutT cvt_out(float v) { return (OutT)v; }

// NM members, LPR lanes per row; rows [rbase, rbase + 4*RP*RITER) of the block
template <int TYPE, int NM, int LPR, typename OutT>
__device__ __forceinline__ void gemv_members(const uint8_t* __restrict__ wexp, int64_t rb, const uint8_t* __restrict__ xq,
                                             int64_t xq_stride, const int* mem, int top_k, int rows, int cols,
                                             OutT* __restrict__ Y, int rbase, const uint32_t* grid) {
  using U = Unit<TYPE>;
  constexpr int RP = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int u0 = lane % LPR;
  const int rsub = lane / LPR;
  const int units = cols / U::VALS;
  const int r0 = rbase + wave * RP * RITER + rsub;
  const uint8_t* xrow[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) xrow[m] = xq + (int64_t)(mem[m] / top_k) * xq_stride;
  float acc[RITER][NM];
#pragma unroll
  for (int i = 0; i < RITER; ++i)
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[i][m] = 0.0f;
  for (int u = u0; u < units; u += LPR) {
    typename U::W w[RITER];
#pragma unroll
    for (int i = 0; i < RITER; ++i) {
      const int r = r0 + i * RP;
      if (r < rows) U::load(wexp + (int64_t)r * rb, u, grid, w[i]);
    }
    int ub0, ub1;
    U::qblocks(u, ub0, ub1);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      Act<U::NQ> a;
      load_act<U::NQ>(xrow[m], ub0, ub1, a);
      U::prep(a);
#pragma unroll
      for (int i = 0; i < RITER; ++i) {
        if (r0 + i * RP < rows) acc[i][m] += U::dot(w[i], a);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RITER; ++i) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      float v = acc[i][m];
#pragma unroll
      for (int mask = LPR / 2; mask > 0; mask >>= 1) v += __shfl_xor(v, mask, 64);
      const int r = r0 + i * RP;
      if (u0 == 0 && r < rows) Y[(int64_t)mem[m] * rows + r] = cvt_out<OutT>(v);
    }
  }
}

template <int TYPE, int LPR, typename OutT>
__global__ __launch_bounds__(256) void moe_gemv_kernel(const uint8_t* __restrict__ xq, int64_t xq_stride,
                                                       const uint8_t* __restrict__ W, int w_is_table,
                                                       int64_t w_expert_stride, const int32_t* __restrict__ ids,
                                                       int top_k, int n_routes, int rows, int cols,
                                                       OutT* __restrict__ Y, int per_route, int n_experts) {
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  constexpr int BR = WAVES * (64 / LPR) * RITER;
  const int p = blockIdx.y;
  const int e = ids[p];
  const int rbase = blockIdx.x * BR;
  if (e < 0 || e >= n_experts) {
    // a route of a CPU expert: zero rows
    for (int r = rbase + threadIdx.x; r < rbase + BR && r < rows; r += blockDim.x) Y[(int64_t)p * rows + r] = cvt_out<OutT>(0.0f);
    return;
  }
  if (!per_route) {
    for (int q = 0; q < p; ++q)
      if (ids[q] == e) return;  // an earlier route of this expert computes this one
  }
  if constexpr (TYPE == GGML_IQ3_S) {
    stage_iq3s_grid(grid);
    __syncthreads();
  }
  const int64_t rb = row_bytes(cols, TYPE);
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W)[e] : W + (int64_t)e * w_expert_stride;
  int q = p;
  while (true) {
    int mem[4];
    int nm = 0;
    if (per_route) {
      if (q != p) break;
      mem[nm++] = p;
      q = n_routes;
    } else {
      for (; q < n_routes && nm < 4; ++q)
        if (ids[q] == e) mem[nm++] = q;
    }
    if (nm == 0) break;
    switch (nm) {
      case 1: gemv_members<TYPE, 1, LPR, OutT>(wexp, rb, xq, xq_stride, mem, top_k, rows, cols, Y, rbase, grid); break;
      case 2: gemv_members<TYPE, 2, LPR, OutT>(wexp, rb, xq, xq_stride, mem, top_k, rows, cols, Y, rbase, grid); break;
      case 3: gemv_members<TYPE, 3, LPR, OutT>(wexp, rb, xq, xq_stride, mem, top_k, rows, cols, Y, rbase, grid); break;
      default: gemv_members<TYPE, 4, LPR, OutT>(wexp, rb, xq, xq_stride, mem, top_k, rows, cols, Y, rbase, grid); break;
    }
    if (per_route) break;
  }
}

template <int TYPE, typename OutT>
int launch_typed(const uint8_t* xq, int64_t xq_stride, const void* W, int w_is_table, int64_t w_expert_stride,
                 const int32_t* ids, int64_t top_k, int64_t n_routes, int64_t rows, int64_t cols, OutT* Y,
                 int per_route, int n_experts, hipStream_t stream) {
  const int units = (int)(cols / Unit<TYPE>::VALS);
  int lpr = 64;
  while (lpr > units) lpr >>= 1;
  if (lpr < 8) lpr = 8;
  const int br = WAVES * (64 / lpr) * RITER;
  dim3 grid((unsigned)((rows + br - 1) / br), (unsigned)n_routes);
  const uint8_t* w = (const uint8_t*)W;
#define KTMI_GEMV_LAUNCH(L)                                                                                        \
  moe_gemv_kernel<TYPE, L, OutT><<<grid, 256, 0, stream>>>(xq, xq_stride, w, w_is_table, w_expert_stride, ids,    \
                                                           (int)top_k, (int)n_routes, (int)rows, (int)cols, Y, \
                                                           per_route, n_experts)
  switch (lpr) {
    case 64: KTMI_GEMV_LAUNCH(64); break;
    case 32: KTMI_GEMV_LAUNCH(32); break;
    case 16: KTMI_GEMV_LAUNCH(16); break;
    default: KTMI_GEMV_LAUNCH(8); break;
  }
#undef KTMI_GEMV_LAUNCH
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

template <typename OutT>
int launch_out(const uint8_t* xq, int64_t xq_stride, const void* W, int w_is_table, int64_t w_expert_stride,
               const int32_t* ids, int64_t top_k, int64_t n_routes, int type, int64_t rows, int64_t cols, OutT* Y,
               int per_route, int n_experts, hipStream_t stream) {
  switch (type) {
    case GGML_Q8_0: return launch_typed<GGML_Q8_0, OutT>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, rows, cols, Y, per_route, n_experts, stream);
    case GGML_Q4_K: return launch_typed<GGML_Q4_K, OutT>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, rows, cols, Y, per_route, n_experts, stream);
    case GGML_Q6_K: return launch_typed<GGML_Q6_K, OutT>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, rows, cols, Y, per_route, n_experts, stream);
    case GGML_IQ3_S: return launch_typed<GGML_IQ3_S, OutT>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, rows, cols, Y, per_route, n_experts, stream);
    default: set_error("moe GEMV: ggml type %d has no kernel", type); return KTMI_ETYPE;
  }
}

}  // namespace

int launch_moe_gemv(const uint8_t* xq, int64_t xq_stride, const void* W, int w_is_table, int64_t w_expert_stride,
                    const int32_t* ids, int64_t top_k, int64_t n_routes, int type, int64_t rows, int64_t cols,
                    void* Y, int y_dtype, int per_route, int n_experts, hipStream_t stream) {
  if (n_routes == 0 || rows == 0) return KTMI_OK;
  switch (y_dtype) {
    case KTMI_F32: return launch_out<float>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, type, rows, cols, (float*)Y, per_route, n_experts, stream);
    case KTMI_F16: return launch_out<_Float16>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, type, rows, cols, (_Float16*)Y, per_route, n_experts, stream);
    case KTMI_BF16: return launch_out<__bf16>(xq, xq_stride, W, w_is_table, w_expert_stride, ids, top_k, n_routes, type, rows, cols, (__bf16*)Y, per_route, n_experts, stream);
    default: set_error("moe GEMV: dtype %d", y_dtype); return KTMI_EINVAL;
  }
}

}  // namespace ktmi
