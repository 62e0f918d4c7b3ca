// Fused decode-sized hot-expert layer (up to DEC_MAX_ROUTES routes): two launches instead
// of the six of the stage-by-stage sequence (quantize x, gate/up GEMV, SiLU*mul, quantize h,
// down GEMV, combine), with the same numerics at every stage boundary:
//
//   decode_gate_up  block (slot e, 32-row group g of the intermediate dim): lists the
//                   routes of slot e, quantises their tokens' x rows to q8_1 in LDS (as
//                   many at a time as fit 64 KB), computes gate rows 32g.. and up rows N+32g.. against them with
//                   the GEMV's units and reduction order, rounds to bf16 (the GEMV output
//                   dtype), applies silu(g)*u in fp32 with one bf16 rounding (sgl-kernel's
//                   silu_and_mul contract, call at hot/kt_gguf_hot.py:260) and writes the
//                   q8_1 block g of each route's h row (kt_gguf_moe_multi.cu:600-650).
//   decode_down     block (8 hidden rows): for every slot with routes (spread over the
//   _combine        waves), the down rows of the block against each route's q8_1 h,
//                   rounded to bf16, kept in LDS; then
//                   the weighted top-k sum in k order (hot/kt_gguf_hot.py:43-71) for the
//                   block's rows of every token. Cold routes contribute nothing (the
//                   reference's zero rows add +0).
//
// Both read every weight byte of a hot slot with routes once per call (the window
// contract of kt_gguf_moe_multi.cu:164-183 at any route count), loading a block's whole
// share of weights into registers before the activations stream past them.
#include "gemv_units.h"
#include "kernels.h"

namespace ktmi {

namespace {

using namespace gemv;

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_RG = 32;     // intermediate rows per gate/up block (one q8_1 block of h)
constexpr int DEC_DR = 8;      // hidden rows per down block
constexpr int DEC_SPW = 4;     // slots per wave and round in the down block (8 lanes per row)
constexpr int DEC_MAX_UNITS = 64;    // gate/up: weight units per row
constexpr int DEC_MCH_MAX = 16;      // member routes per pass of the gate/up block, at most
constexpr int DEC_MCH_CHUNK = 8;     // member routes per gate/up block and pass
constexpr int DEC_MAX_UNITS2 = 16;   // down: weight units per row

__device__ __forceinline__ float bf16_round(float v) { return (float)(__bf16)v; }

// sum over aligned groups of L = 8 or 16 lanes, the same value in every lane of a group:
// DPP xor-1 and xor-2 inside quads, then the mirror of each 8-lane half row (and of the
// 16-lane row for L = 16); float addition commutes, so partner lanes agree bit for bit
template <int CTRL>
__device__ __forceinline__ float dpp_plus(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false);
  return v + __int_as_float(o);
}
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(L == 8 || L == 16, "group size");
  v = dpp_plus<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_plus<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_plus<0x141>(v);  // row_half_mirror
  if constexpr (L == 16) v = dpp_plus<0x140>(v);  // row_mirror
  return v;
}

// lanes per row of the down block: 8, or 16 for rows of 16 units (each lane one unit)
__host__ __device__ constexpr int dec_lpr(int units) { return units >= 16 ? 16 : 8; }

// One block per (slot e, group g of 32 intermediate rows, member chunk z): 512 threads = 64
// rows (32 gate rows 32g.., 32 up rows N+32g..) x 8 lanes; lane j of a row holds units j,
// j+8, ... of it (UPL of them). Every weight unit is loaded into registers before any
// activation is touched, then the block's member routes (routes of slot e; chunks z,
// z + gridDim.z, ... of mch routes) stream past them. Splitting a popular slot's routes
// over gridDim.z blocks keeps its rows from serialising the kernel.
template <int TYPE, int UPL>
__global__ __launch_bounds__(DEC_THREADS) void decode_gate_up(const __bf16* __restrict__ x, int K, int N,
                                                              const int32_t* __restrict__ slot_ids, int top_k, int R,
                                                              int S, const uint8_t* __restrict__ W13, int w_is_table,
                                                              int64_t w_stride, uint8_t* __restrict__ hq,
                                                              int64_t hq_stride, int mch) {
  using U = Unit<TYPE>;
  constexpr int LPR = 8;
  static_assert(DEC_THREADS / LPR == 2 * DEC_RG, "one row per thread group");
  extern __shared__ __attribute__((aligned(16))) uint8_t xq_lds[];  // mch q8_1 rows of K
  __shared__ int mem[DEC_MAX_ROUTES];
  __shared__ int wcnt[DEC_WAVES];
  __shared__ float gu[DEC_MCH_MAX][2 * DEC_RG];
  __shared__ int2 xs_lds[DEC_MCH_MAX * DEC_MAX_UNITS * 2];  // int8 sums of q8_1 half-blocks
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  const int e = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x;
  // the routes of slot e in ascending order (every block of the slot sees the same list,
  // so the member chunks split over gridDim.z are disjoint): thread p tests route p
  static_assert(DEC_MAX_ROUTES <= DEC_THREADS, "one route per thread");
  const int lane = tid & 63, wv = tid >> 6;
  const bool hit = tid < R && slot_ids[tid] == e;
  const uint64_t bal = __ballot(hit);
  if (lane == 0) wcnt[wv] = __popcll(bal);
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  __syncthreads();
  int base = 0, nm = 0;
#pragma unroll
  for (int k = 0; k < DEC_WAVES; ++k) {
    base += k < wv ? wcnt[k] : 0;
    nm += wcnt[k];
  }
  if (hit) mem[base + __popcll(bal & ((1ull << lane) - 1))] = tid;
  __syncthreads();
  const int cz = blockIdx.z, nz = gridDim.z;
  if (cz * mch >= nm) return;  // uniform: no route of this slot (or of this chunk)
  const int64_t rb = row_bytes(K, TYPE);
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W13)[e] : W13 + (int64_t)e * w_stride;
  const int i = tid / LPR, j0 = tid % LPR;
  const int row = i < DEC_RG ? g * DEC_RG + i : N + g * DEC_RG + (i - DEC_RG);
  const uint8_t* wrow = wexp + (int64_t)row * rb;
  const int units = K / U::VALS;
  const int Kp = (int)q8_1_cols_padded(K);
  const int xq_row = Kp / 32 * QB8_1;
  const int KB = Kp / 32;  // q8_1 blocks per row; mch * KB <= DEC_THREADS: one block per thread
  // q8_1 of the members' x rows, one thread per 32-value block (d and q as the quantize_q8_1
  // kernel; the header's fp16 sum field, which no unit reads, is summed in index order here).
  // Split in two so the first chunk's x loads go out before the weight loads, and the
  // weights are unpacked only after the quantisation.
  u32x4_t xr[4];
  auto load_x = [&](int c0, int nc) {
    const int m = tid / KB, kb = tid % KB;
    if (m < nc && kb * 32 < K) {
      const __bf16* src = x + (int64_t)(mem[c0 + m] / top_k) * K + kb * 32;
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[c] = gload<u32x4_t>(src + 8 * c);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) xr[c] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto quantize_x = [&](int nc) {
    const int m = tid / KB, kb = tid % KB;
    if (m >= nc) return;
    int2 hs = {0, 0};
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[8 * c + 2 * t] = __uint_as_float(xr[c][t] << 16);
        v[8 * c + 2 * t + 1] = __uint_as_float(xr[c][t] & 0xFFFF0000u);
      }
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      amax = fmaxf(amax, fabsf(v[t]));
      sum += v[t];
    }
    const float d = amax / 127.0f;
    uint8_t* blk = xq_lds + m * xq_row + kb * QB8_1;
    *(uint32_t*)blk = (uint32_t)float_to_half_bits(d) | ((uint32_t)float_to_half_bits(sum) << 16);
#pragma unroll
    for (int q8 = 0; q8 < 8; ++q8) {
      uint32_t wd = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int8_t q = amax == 0.0f ? 0 : (int8_t)roundf(v[4 * q8 + t] / d);
        wd |= (uint32_t)(uint8_t)q << (8 * t);
        if (q8 < 4) hs.x += q; else hs.y += q;
      }
      *(uint32_t*)(blk + 4 + 4 * q8) = wd;
    }
    xs_lds[m * KB + kb] = hs;
  };
  load_x(cz * mch, min(mch, nm - cz * mch));
  __builtin_amdgcn_sched_barrier(0);
  typename U::W w[UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j)
    if (j0 + LPR * j < units) U::load(wrow, j0 + LPR * j, grid, w[j]);
  __builtin_amdgcn_sched_barrier(0);
  quantize_x(min(mch, nm - cz * mch));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < UPL; ++j)
    if (j0 + LPR * j < units) U::finish(w[j], grid);
  for (int c0 = cz * mch; c0 < nm; c0 += nz * mch) {
    const int nc = min(mch, nm - c0);
    if (c0 > cz * mch) {
      load_x(c0, nc);
      quantize_x(nc);
    }
    __syncthreads();
    for (int m = 0; m < nc; ++m) {
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < UPL; ++j) {
        const int u = j0 + LPR * j;
        if (u < units) {
          int ub0, ub1;
          U::qblocks(u, ub0, ub1);
          Act<U::NQ> a;
          load_act<U::NQ>(xq_lds + m * xq_row, ub0, ub1, a);
          // the int8 sums the units need (Unit::prep), computed once per block in quantize_x
          const int2 s0 = xs_lds[m * KB + ub0], s1 = xs_lds[m * KB + ub1];
          if constexpr (TYPE == GGML_Q4_K) {
            a.s[0] = s0.x + s0.y;
            a.s[1] = s1.x + s1.y;
          } else if constexpr (TYPE == GGML_Q6_K) {
            a.s[0] = s0.x;
            a.s[1] = s0.y;
            a.s[2] = s1.x;
            a.s[3] = s1.y;
          }
          v += U::dot(w[j], a);
        }
      }
      v = group_sum<LPR>(v);
      if (j0 == 0) gu[m][i] = bf16_round(v);  // the GEMV's bf16 output
    }
    __syncthreads();
    // silu(g)*u in fp32, one bf16 rounding, then q8_1 block g of each member's h row
    for (int idx = tid; idx < nc * 32; idx += DEC_THREADS) {
      const int m = idx / 32, t = idx % 32;
      const float gg = gu[m][t], uu = gu[m][DEC_RG + t];
      const float hv = bf16_round(gg / (1.0f + expf(-gg)) * uu);
      float amax = fabsf(hv);
      float sum = hv;
#pragma unroll
      for (int mask = 16; mask > 0; mask >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, mask, 32));
        sum += __shfl_xor(sum, mask, 32);
      }
      const float d = amax / 127.0f;
      const int8_t q = amax == 0.0f ? 0 : (int8_t)roundf(hv / d);
      uint8_t* blk = hq + (int64_t)mem[c0 + m] * hq_stride + g * QB8_1;
      blk[4 + t] = (uint8_t)q;
      if (t == 0) *(uint32_t*)blk = (uint32_t)float_to_half_bits(d) | ((uint32_t)float_to_half_bits(sum) << 16);
    }
    __syncthreads();
  }
}

// One block per DEC_DR hidden rows. The hot routes are grouped by slot in LDS; wave w takes
// the slots with routes w, w + DEC_WAVES, ... (DEC_SPW per round), loads the block's rows of
// all of them into registers first, then runs every route of each past them. Y (bf16, the
// GEMV output dtype) stays in LDS; the block ends with the weighted top-k sum of its rows.
template <int TYPE, int LPR>
__global__ __launch_bounds__(DEC_THREADS) void decode_down_combine(const uint8_t* __restrict__ hq, int64_t hq_stride,
                                                                   int K, int N, const int32_t* __restrict__ slot_ids,
                                                                   const float* __restrict__ topk_w, int T, int top_k,
                                                                   int S, const uint8_t* __restrict__ W2,
                                                                   int w_is_table, int64_t w_stride,
                                                                   __bf16* __restrict__ y) {
  using U = Unit<TYPE>;
  constexpr int RPW = 64 / LPR;         // rows per wave pass
  constexpr int RIT = DEC_DR / RPW;     // passes over the block's rows
  constexpr int SPW = DEC_SPW / RIT;    // slots per wave and round (registers: SPW * RIT units)
  static_assert(RIT >= 1 && DEC_DR % RPW == 0 && SPW >= 1, "row split");
  __shared__ int cnt[DEC_MAX_SLOTS + 1];
  __shared__ int act_slots[DEC_MAX_SLOTS];
  __shared__ int n_act_s;
  __shared__ int order[DEC_MAX_ROUTES];   // hot routes grouped by slot
  __shared__ int pos_of[DEC_MAX_ROUTES];  // route -> index in order (-1: not hot)
  __shared__ float yv[DEC_MAX_ROUTES][DEC_DR];
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int R = T * top_k;
  const int c0 = blockIdx.x * DEC_DR;
  // counting sort of the hot routes by slot (the order inside a slot is irrelevant: every
  // route's row sums are independent)
  for (int i = tid; i <= S; i += DEC_THREADS) cnt[i] = 0;
  if (tid == 0) n_act_s = 0;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  __syncthreads();
  for (int p = tid; p < R; p += DEC_THREADS) {
    const int e = slot_ids[p];
    if (e >= 0 && e < S) atomicAdd(&cnt[e + 1], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int n = 0;
    for (int i = 1; i <= S; ++i) {
      if (cnt[i] > 0) act_slots[n++] = i - 1;
      cnt[i] += cnt[i - 1];
    }
    n_act_s = n;
  }
  __syncthreads();
  for (int p = tid; p < R; p += DEC_THREADS) {
    const int e = slot_ids[p];
    int at = -1;
    if (e >= 0 && e < S) {
      at = atomicAdd(&cnt[e], 1);  // cnt[e] runs from the slot's start to its end
      order[at] = p;
    }
    pos_of[p] = at;
  }
  __syncthreads();
  // cnt[e] is now the end of slot e's run and cnt[e - 1] its start (0 for e == 0)
  const int n_act = n_act_s;
  const int64_t rb = row_bytes(N, TYPE);
  const int u = lane % LPR;
  const bool ulive = u < N / U::VALS;
  int ub0, ub1;
  U::qblocks(u, ub0, ub1);
  for (int base = 0; base < n_act; base += DEC_WAVES * SPW) {
    typename U::W w[SPW][RIT];
    int sl[SPW];
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int k = base + wave + DEC_WAVES * j;
      sl[j] = k < n_act ? act_slots[k] : -1;
      if (sl[j] >= 0 && ulive) {
        const int e = sl[j];
        const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W2)[e] : W2 + (int64_t)e * w_stride;
#pragma unroll
        for (int r = 0; r < RIT; ++r) U::load(wexp + (int64_t)(c0 + r * RPW + lane / LPR) * rb, u, grid, w[j][r]);
      }
    }

#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (sl[j] < 0) continue;  // uniform per wave
      if (ulive)
#pragma unroll
        for (int r = 0; r < RIT; ++r) U::finish(w[j][r], grid);  // the others' loads stay in flight
      const int e = sl[j];
      const int beg = e == 0 ? 0 : cnt[e - 1], end = cnt[e];
      // two routes at a time: both activation loads are in flight together
      for (int at = beg; at < end; at += 2) {
        const bool two = at + 1 < end;
        Act<U::NQ> a[2];
        if (ulive) {
          load_act<U::NQ>(hq + (int64_t)order[at] * hq_stride, ub0, ub1, a[0]);
          load_act<U::NQ>(hq + (int64_t)order[two ? at + 1 : at] * hq_stride, ub0, ub1, a[1]);
          U::prep(a[0]);
          U::prep(a[1]);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          if (m == 1 && !two) break;  // uniform per wave
#pragma unroll
          for (int r = 0; r < RIT; ++r) {
            const float v = group_sum<LPR>(ulive ? U::dot(w[j][r], a[m]) : 0.0f);
            if (u == 0) yv[at + m][r * RPW + lane / LPR] = bf16_round(v);
          }
        }
      }
    }
  }
  __syncthreads();
  // res[t, c] = bf16(sum over k ascending of bf16(Y[t,k,c] * bf16(w[t,k])))
  for (int q = tid; q < T * DEC_DR; q += DEC_THREADS) {
    const int t = q / DEC_DR, i = q % DEC_DR;
    float acc = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      const int at = pos_of[t * top_k + k];
      if (at < 0) continue;
      const float wk = bf16_round(topk_w[t * top_k + k]);
      acc += bf16_round(yv[at][i] * wk);
    }
    y[(int64_t)t * K + c0 + i] = (__bf16)acc;
  }
}

template <int TYPE>
int launch_gate_up(const __bf16* x, int64_t K, int64_t N, const int32_t* slot_ids, int64_t top_k, int64_t R,
                   int64_t S, const uint8_t* W13, int w_is_table, int64_t w_stride, uint8_t* hq, int64_t hq_stride,
                   hipStream_t stream) {
  const int64_t xq_row = q8_1_row_bytes(K);
  int mch = (int)(DEC_MAX_XQ_LDS / xq_row < DEC_MCH_CHUNK ? DEC_MAX_XQ_LDS / xq_row : DEC_MCH_CHUNK);
  const int kb = (int)(q8_1_cols_padded(K) / 32);
  if (mch * kb > DEC_THREADS) mch = DEC_THREADS / kb;  // one q8_1 block per thread and chunk
  const size_t lds = (size_t)mch * (size_t)xq_row;
  // one block per row group walks all of a slot's routes: splitting them over more blocks
  // (gridDim.z) re-reads the weights once per extra block, which costs more than it saves
  // at decode sizes
  dim3 grid((unsigned)S, (unsigned)(N / DEC_RG), 1);
#define KTMI_GU(P)                                                                                          \
  decode_gate_up<TYPE, P><<<grid, DEC_THREADS, lds, stream>>>(x, (int)K, (int)N, slot_ids, (int)top_k, (int)R, \
                                                               (int)S, W13, w_is_table, w_stride, hq, hq_stride, mch)
  const int64_t units = K / Unit<TYPE>::VALS;  // <= DEC_MAX_UNITS: decode_layer_fits
  if (units <= 8) KTMI_GU(1);
  else if (units <= 16) KTMI_GU(2);
  else if (units <= 32) KTMI_GU(4);
  else KTMI_GU(8);
#undef KTMI_GU

  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

template <int TYPE>
int launch_down(const uint8_t* hq, int64_t hq_stride, int64_t K, int64_t N, const int32_t* slot_ids,
                const float* topk_w, int64_t T, int64_t top_k, int64_t S, const uint8_t* W2, int w_is_table,
                int64_t w_stride, __bf16* y, hipStream_t stream) {
  const unsigned nb = (unsigned)(K / DEC_DR);
#define KTMI_DN(L)                                                                                          \
  decode_down_combine<TYPE, L><<<nb, DEC_THREADS, 0, stream>>>(hq, hq_stride, (int)K, (int)N, slot_ids, topk_w, \
                                                              (int)T, (int)top_k, (int)S, W2, w_is_table,     \
                                                              w_stride, y)
  switch (dec_lpr((int)(N / Unit<TYPE>::VALS))) {  // <= 16 units: decode_layer_fits
    case 16: KTMI_DN(16); break;
    default: KTMI_DN(8); break;
  }
#undef KTMI_DN
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

int unit_vals(int type) { return type == GGML_Q4_K || type == GGML_Q6_K ? 64 : 32; }

}  // namespace

bool decode_layer_fits(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  // every lane holds at most one weight unit of a row; the down block's registers hold
  // 4 row units of up to 16 lanes each
  return tokens * top_k <= DEC_MAX_ROUTES && L->n_slots <= DEC_MAX_SLOTS && L->inter % DEC_RG == 0 &&
         L->hidden % DEC_DR == 0 && q8_1_row_bytes(L->hidden) <= DEC_MAX_XQ_LDS &&
         L->hidden / unit_vals(L->type13) <= DEC_MAX_UNITS && L->inter / unit_vals(L->type2) <= DEC_MAX_UNITS2;
}

int64_t decode_layer_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  return (tokens * top_k * q8_1_row_bytes(L->inter) + 255) & ~(int64_t)255;
}

int launch_decode_layer(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                        int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots, R = tokens * top_k;
  const int64_t hq_stride = q8_1_row_bytes(N);
  const uint8_t* W13 = (const uint8_t*)L->w13;
  const uint8_t* W2 = (const uint8_t*)L->w2;
  const int64_t st13 = 2 * N * row_bytes(K, L->type13), st2 = K * row_bytes(N, L->type2);
  record_stage(0, stream);
  record_stage(1, stream);
  int rc;
  switch (L->type13) {
    case GGML_Q8_0: rc = launch_gate_up<GGML_Q8_0>((const __bf16*)x, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_Q4_K: rc = launch_gate_up<GGML_Q4_K>((const __bf16*)x, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_Q6_K: rc = launch_gate_up<GGML_Q6_K>((const __bf16*)x, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_IQ3_S: rc = launch_gate_up<GGML_IQ3_S>((const __bf16*)x, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    default: set_error("decode layer: ggml type %d has no kernel", L->type13); return KTMI_ETYPE;
  }
  if (rc) return rc;
  record_stage(2, stream);
  record_stage(3, stream);
  switch (L->type2) {
    case GGML_Q8_0: rc = launch_down<GGML_Q8_0>(ws, hq_stride, K, N, slot_ids, topk_w, tokens, top_k, S, W2, L->w_is_table, st2, (__bf16*)y, stream); break;
    case GGML_Q4_K: rc = launch_down<GGML_Q4_K>(ws, hq_stride, K, N, slot_ids, topk_w, tokens, top_k, S, W2, L->w_is_table, st2, (__bf16*)y, stream); break;
    case GGML_Q6_K: rc = launch_down<GGML_Q6_K>(ws, hq_stride, K, N, slot_ids, topk_w, tokens, top_k, S, W2, L->w_is_table, st2, (__bf16*)y, stream); break;
    case GGML_IQ3_S: rc = launch_down<GGML_IQ3_S>(ws, hq_stride, K, N, slot_ids, topk_w, tokens, top_k, S, W2, L->w_is_table, st2, (__bf16*)y, stream); break;
    default: set_error("decode layer: ggml type %d has no kernel", L->type2); return KTMI_ETYPE;
  }
  record_stage(4, stream);
  record_stage(5, stream);
  return rc;
}

}  // namespace ktmi
