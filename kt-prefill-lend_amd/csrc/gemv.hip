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
#include "gemv_units.h"
#include "kernels.h"

namespace ktmi {

namespace {

constexpr int RITER = 4;
constexpr int WAVES = 4;
using namespace gemv;

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
#pragma unroll
    for (int i = 0; i < RITER; ++i)
      if (r0 + i * RP < rows) U::finish(w[i], grid);
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
