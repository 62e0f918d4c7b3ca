// Fused decode-sized hot-expert layer (up to DEC_MAX_ROUTES routes): two launches instead
// of the six of the stage-by-stage sequence (quantize x, gate/up GEMV, SiLU*mul, quantize h,
// down GEMV, combine) -- three from DEC_PREQ_TOKENS tokens on, where x is quantised by its
// own launch -- with the same numerics at every stage boundary:
//
//   decode_gate_up  block (k-th slot with routes, 32-row group g of the intermediate dim):
//                   lists the routes of the slot, quantises their tokens' x rows to q8_1 in
//                   LDS (or loads the q8_1 rows of x quantised by the launch before),
//                   computes gate rows 32g.. and up rows N+32g.. against them with the
//                   GEMV's units, rounds to bf16 (the GEMV output dtype), applies
//                   silu(g)*u in fp32 with one bf16 rounding (sgl-kernel's silu_and_mul
//                   contract, call at hot/kt_gguf_hot.py:260) and writes the q8_1 block g of
//                   each route's h row (kt_gguf_moe_multi.cu:600-650).
//   decode_down     block (8 hidden rows): the hot routes grouped by slot, their q8_1 h rows
//   _combine        staged in LDS with one round of loads; for every slot with routes
//                   (spread over the waves), the down rows of the block against each
//                   route's h, rounded to bf16 and kept in LDS; then the weighted top-k sum
//                   in k order (hot/kt_gguf_hot.py:43-71) for the block's rows of every
//                   token. Cold routes contribute nothing (the reference's zero rows add +0).
//
// Both read every weight byte of a hot slot with routes once per call (the window
// contract of kt_gguf_moe_multi.cu:164-183 at any route count), loading a block's whole
// share of weights into registers before the activations stream past them. Slots without
// routes cost no block: gate/up blocks are numbered over the slots that have routes (the
// last blocks of the grid exit at once), with the row group fastest so that one slot's
// groups spread over all XCDs (consecutive blocks go to consecutive XCDs).
#include <type_traits>

#include "gemv_units.h"
#include "kernels.h"

namespace ktmi {

namespace {

using namespace gemv;

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_RG = 32;     // intermediate rows per gate/up block (one q8_1 block of h)
constexpr int DEC_GLPR = 16;   // gate/up: lanes per intermediate row (its gate and up rows)
constexpr int DEC_DR = 8;      // hidden rows per down block
constexpr int DEC_SPW = 4;     // slots per wave and round in the down block (8 lanes per row)
constexpr int DEC_MAX_UNITS = 64;    // gate/up: weight units per row
constexpr int DEC_MCH_MAX = 16;      // member routes per pass of the gate/up block, at most
constexpr int DEC_XQB = 2 * DEC_THREADS;  // gate/up: q8_1 blocks of x per pass, at most
constexpr int DEC_XRAW_LDS = 64 * 1024;   // gate/up: the pass's bf16 x rows
constexpr int DEC_PREQ_TOKENS = 8;        // from this many tokens on, x is quantised by its own launch
constexpr int DEC_MAX_UNITS2 = 16;   // down: weight units per row
constexpr int DEC_HL_LDS = 80 * 1024;                   // down: staged q8_1 h rows
static_assert(DEC_MAX_SLOTS <= DEC_THREADS && DEC_MAX_ROUTES <= DEC_THREADS, "one slot and one route per thread");

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

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false);
  return fmaxf(v, __int_as_float(o));
}
template <int CTRL>
__device__ __forceinline__ int dpp_iadd(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// The GEMV units with the weight bits unpacked once per weight load rather than once per
// route: Q4_K keeps its low and high nibbles apart, Q6_K its 6-bit values (nibble | 2 high
// bits << 4) for both halves. The integer sums are those of Unit<TYPE>::dot.
template <int TYPE>
struct DUnit : Unit<TYPE> {};

template <>
struct DUnit<GGML_Q4_K> : Unit<GGML_Q4_K> {
  using B = Unit<GGML_Q4_K>;
  struct W { B::W b; uint32_t lo[8], hi[8]; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t* grid, W& w) { B::load(row, u, grid, w.b); }
  __device__ static void finish(W& w, const uint32_t* grid) {
    B::finish(w.b, grid);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w.lo[i] = w.b.q[i] & 0x0F0F0F0Fu;
      w.hi[i] = (w.b.q[i] >> 4) & 0x0F0F0F0Fu;
    }
  }
  __device__ static float dot(const W& w, const Act<2>& a) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s0 = dot4(w.lo[i], a.q[i], s0);
      s1 = dot4(w.hi[i], a.q[8 + i], s1);
    }
    const float sd = a.d[0] * (float)(s0 * w.b.sc0) + a.d[1] * (float)(s1 * w.b.sc1);
    const float sm = a.d[0] * (float)(a.s[0] * w.b.m0) + a.d[1] * (float)(a.s[1] * w.b.m1);
    return w.b.d * sd - w.b.dmin * sm;
  }
};

template <>
struct DUnit<GGML_Q6_K> : Unit<GGML_Q6_K> {
  using B = Unit<GGML_Q6_K>;
  struct W { B::W b; uint32_t lo[8], hi[8]; };
  __device__ static void load(const uint8_t* row, int u, const uint32_t* grid, W& w) { B::load(row, u, grid, w.b); }
  __device__ static void finish(W& w, const uint32_t* grid) {
    B::finish(w.b, grid);
    const int sh = 2 * w.b.c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w.lo[i] = (w.b.ql[i] & 0x0F0F0F0Fu) | (((w.b.qh[i] >> sh) & 0x03030303u) << 4);
      w.hi[i] = ((w.b.ql[i] >> 4) & 0x0F0F0F0Fu) | (((w.b.qh[i] >> (sh + 4)) & 0x03030303u) << 4);
    }
  }
  __device__ static float dot(const W& w, const Act<2>& a) {
    int s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s[i >> 2] = dot4(w.lo[i], a.q[i], s[i >> 2]);
      s[2 + (i >> 2)] = dot4(w.hi[i], a.q[8 + i], s[2 + (i >> 2)]);
    }
    const float p0 = (float)(w.b.sc[0] * (s[0] - 32 * a.s[0]) + w.b.sc[1] * (s[1] - 32 * a.s[1]));
    const float p1 = (float)(w.b.sc[2] * (s[2] - 32 * a.s[2]) + w.b.sc[3] * (s[3] - 32 * a.s[3]));
    return w.b.d * (a.d[0] * p0 + a.d[1] * p1);
  }
};

// the int8 sums a unit needs of its activation blocks (Unit::prep), from the int2 half-block
// sums (values 0-15, 16-31) of q8_1 blocks ub0 and ub1
template <int TYPE, int NQ>
__device__ __forceinline__ void act_sums(Act<NQ>& a, int2 s0, int2 s1) {
  if constexpr (TYPE == GGML_Q4_K) {
    a.s[0] = s0.x + s0.y;
    a.s[1] = s1.x + s1.y;
  } else if constexpr (TYPE == GGML_Q6_K) {
    a.s[0] = s0.x;
    a.s[1] = s0.y;
    a.s[2] = s1.x;
    a.s[3] = s1.y;
  }
}
constexpr bool needs_sums(int type) { return type == GGML_Q4_K || type == GGML_Q6_K; }

// q8_1 of 32 bf16 values spread over an aligned group of 8 lanes, 4 values (two packed bf16
// pairs) a lane: d = amax / 127 and q = round(v / d) as the quantize_q8_1 kernel (the
// header's fp16 sum field is left 0: no unit reads it). Writes the block at blk and, from
// lane 0 of the group, the int2 half-block sums (values 0-15, 16-31) to *hs.
__device__ __forceinline__ void quantize_q8_1_x8(u32x2_t xv, int part, uint8_t* blk, int2* hs) {
  const float v[4] = {__uint_as_float(xv[0] << 16), __uint_as_float(xv[0] & 0xFFFF0000u),
                      __uint_as_float(xv[1] << 16), __uint_as_float(xv[1] & 0xFFFF0000u)};
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = dpp_max<0xB1>(amax);   // quad_perm [1,0,3,2]
  amax = dpp_max<0x4E>(amax);   // quad_perm [2,3,0,1]
  amax = dpp_max<0x141>(amax);  // row_half_mirror: the 8-lane group
  const float d = amax / 127.0f;
  uint32_t wd = 0;
  int qs = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int8_t q = amax == 0.0f ? 0 : (int8_t)roundf(v[t] / d);
    wd |= (uint32_t)(uint8_t)q << (8 * t);
    qs += q;
  }
  *(uint32_t*)(blk + 4 + 4 * part) = wd;
  qs = dpp_iadd<0xB1>(qs);
  qs = dpp_iadd<0x4E>(qs);  // the quad's sum in every lane of it
  const int other = __builtin_amdgcn_update_dpp(0, qs, 0x141, 0xF, 0xF, false);  // lane 0 <- lane 7
  if (part == 0) {
    *(uint32_t*)blk = (uint32_t)float_to_half_bits(d);
    *hs = int2{qs, other};
  }
}

// exclusive prefix sum over the DEC_THREADS threads of the block (one value each); every
// thread gets the total too. Uses wsum[DEC_WAVES]; ends with the block synchronised.
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, 64);
    if (lane >= o) inc += t;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < DEC_WAVES; ++k) {
    const int s = wsum[k];
    before += k < wv ? s : 0;
    total += s;
  }
  return before + inc - v;
}

__device__ __forceinline__ int lanes_below(uint64_t bal) {
  return __popcll(bal & ((1ull << (threadIdx.x & 63)) - 1));
}

// lanes per row of the down block: 8, or 16 for rows of 16 units (each lane one unit)
__host__ __device__ constexpr int dec_lpr(int units) { return units >= 16 ? 16 : 8; }

// The block's slot and its routes: blocks are numbered k * G + g over the slots that have
// routes (ascending), so block kslot serves the kslot-th of them. Leaves the slot's routes in
// ascending order in mem[0 .. nm) and returns false (for the whole block) when fewer than
// kslot + 1 slots have routes. Thread p tests route p (R <= DEC_MAX_ROUTES <= DEC_THREADS).
__device__ __forceinline__ bool slot_members(const int32_t* __restrict__ slot_ids, int R, int S, int kslot,
                                             uint8_t* present, int (*wsum)[DEC_WAVES], int* sel, int* mem, int& e,
                                             int& nm) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  present[tid] = 0;  // DEC_MAX_SLOTS <= DEC_THREADS entries
  const int sid = tid < R ? slot_ids[tid] : -1;
  __syncthreads();
  if (sid >= 0 && sid < S) present[sid] = 1;
  __syncthreads();
  const bool pres = present[tid] != 0;
  const uint64_t pb = __ballot(pres);
  if (lane == 0) wsum[0][wv] = __popcll(pb);
  __syncthreads();
  int before = 0, n_act = 0;
#pragma unroll
  for (int k = 0; k < DEC_WAVES; ++k) {
    before += k < wv ? wsum[0][k] : 0;
    n_act += wsum[0][k];
  }
  if (kslot >= n_act) return false;  // uniform
  if (pres && before + lanes_below(pb) == kslot) *sel = tid;
  __syncthreads();
  e = *sel;
  const bool hit = sid == e;
  const uint64_t bal = __ballot(hit);
  if (lane == 0) wsum[1][wv] = __popcll(bal);
  __syncthreads();
  int base = 0;
  nm = 0;
#pragma unroll
  for (int k = 0; k < DEC_WAVES; ++k) {
    base += k < wv ? wsum[1][k] : 0;
    nm += wsum[1][k];
  }
  if (hit) mem[base + lanes_below(bal)] = tid;
  __syncthreads();
  return true;
}

// silu(g)*u in fp32 with one bf16 rounding from the bf16 GEMV outputs gu[m][0..32) (gate
// rows) and gu[m][32..64) (up rows), then q8_1 block g of each of the nc members' h rows
__device__ __forceinline__ void silu_h_q8_1(const float (*gu)[2 * DEC_RG], int nc, const int* mem, uint8_t* hq,
                                            int64_t hq_stride, int g) {
  for (int idx = threadIdx.x; idx < nc * 32; idx += DEC_THREADS) {
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
    uint8_t* blk = hq + (int64_t)mem[m] * hq_stride + g * QB8_1;
    blk[4 + t] = (uint8_t)q;
    if (t == 0) *(uint32_t*)blk = (uint32_t)float_to_half_bits(d) | ((uint32_t)float_to_half_bits(sum) << 16);
  }
}

// One block per (k-th slot with routes, group g of 32 intermediate rows), numbered k * G + g
// (G = N / 32 groups): 512 threads = 32 intermediate rows x 16 lanes; lane j of row i holds
// units j, j+16, ... (UPL of them) of gate row 32g+i and of up row N+32g+i, so every
// activation read serves both. Every weight unit is loaded into registers before any
// activation is touched; then the member routes (the routes of the slot, ascending, mch
// per pass) stream past them. With PREQ, x arrives already as q8_1 rows (xq, quantised once
// per token by the quantize_q8_1 kernel): every block of a slot would otherwise repeat the
// quantisation of the slot's tokens, the largest cost of the popular slots' blocks once a
// window holds more than a few tokens.
template <int TYPE, int UPL, bool PREQ>
__global__ __launch_bounds__(DEC_THREADS) void decode_gate_up(const __bf16* __restrict__ x, int K, int N,
                                                                 const int32_t* __restrict__ slot_ids, int top_k,
                                                                 int R, int S, const uint8_t* __restrict__ W13,
                                                                 int w_is_table, int64_t w_stride,
                                                                 uint8_t* __restrict__ hq, int64_t hq_stride,
                                                                 int mch, const uint8_t* __restrict__ xq) {
  // four units a lane (K above 2048 for the 64-value units) leave no registers for unpacked bits
  using U = std::conditional_t<UPL <= 2, DUnit<TYPE>, Unit<TYPE>>;
  constexpr int LPR = DEC_GLPR;
  static_assert(DEC_THREADS / LPR == DEC_RG, "one intermediate row per lane group");
  extern __shared__ __attribute__((aligned(16))) uint8_t xq_lds[];  // mch q8_1 rows of K
  __shared__ int mem[DEC_MAX_ROUTES];
  __shared__ int wsum[2][DEC_WAVES];
  __shared__ int sel;
  __shared__ uint8_t present[DEC_MAX_SLOTS];
  __shared__ float gu[DEC_MCH_MAX][2 * DEC_RG];
  __shared__ int2 xs_lds[DEC_XQB];  // int8 sums of the q8_1 half-blocks
  // the pass's x rows as they are in HBM (bf16), one 64-piece wave load past the last row
  __shared__ __attribute__((aligned(16))) uint8_t xraw[PREQ ? 16 : DEC_XRAW_LDS + 1024];
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = N / DEC_RG;
  const int kslot = blockIdx.x / G, g = blockIdx.x % G;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  int e, nm;
  if (!slot_members(slot_ids, R, S, kslot, present, wsum, &sel, mem, e, nm)) return;
  const int64_t rb = row_bytes(K, TYPE);
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W13)[e] : W13 + (int64_t)e * w_stride;
  const int i = tid / LPR, j0 = tid % LPR;
  const uint8_t* wg = wexp + (int64_t)(g * DEC_RG + i) * rb;
  const uint8_t* wu = wexp + (int64_t)(N + g * DEC_RG + i) * rb;
  const int units = K / U::VALS;
  const int Kp = (int)q8_1_cols_padded(K);
  const int xq_row = Kp / 32 * QB8_1;
  const int KB = Kp / 32;  // q8_1 blocks per row; mch * KB <= DEC_XQB, mch * K * 2 <= DEC_XRAW_LDS
  // x rows of a pass's members: buffer loads straight into LDS (16 bytes a lane, piece q of
  // the pass at xraw + 16 q), then q8_1 from there with 8 lanes per 32-value block. Loops,
  // not unrolled copies: at decode sizes each block runs through its code about once. With
  // PREQ the q8_1 rows themselves are loaded into xq_lds and only their half-block sums
  // are formed here.
  const int ppr = PREQ ? xq_row / 16 : K / 8;  // 16-byte pieces per row
  const int T = R / top_k;
  const uint32_t x_bytes = PREQ ? (uint32_t)T * (uint32_t)xq_row : (uint32_t)T * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t x_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(PREQ ? (void*)xq : (void*)x, (short)0, x_bytes, 0x00020000);
  uint8_t* xdst = PREQ ? xq_lds : xraw;
  auto load_x = [&](int c0, int nc) {
    const int nq = nc * ppr;
    const uint32_t row_bytes_x = PREQ ? (uint32_t)xq_row : (uint32_t)K * 2u;
    for (int q0 = wv * 64; q0 < nq; q0 += DEC_THREADS) {  // uniform per wave
      const int q = q0 + lane, m = q / ppr;
      const uint32_t off = q < nq ? (uint32_t)(mem[c0 + m] / top_k) * row_bytes_x + (uint32_t)(q - m * ppr) * 16u : x_bytes;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rsrc, (__attribute__((address_space(3))) void*)(xdst + q0 * 16), 16,
                                               (int)off, 0, 0, 0);
    }
  };
  auto quantize_x = [&](int nc) {
    if constexpr (PREQ) {
      for (int blk = tid; blk < nc * KB; blk += DEC_THREADS) {  // blk == m * KB + kb: row m at m * xq_row
        const uint32_t* qw = (const uint32_t*)(xq_lds + blk * QB8_1 + 4);
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo = dot4(0x01010101u, qw[i], lo);
          hi = dot4(0x01010101u, qw[4 + i], hi);
        }
        xs_lds[blk] = int2{lo, hi};
      }
    } else {
      const int nt = nc * KB * 8;
      for (int q = tid; q < nt; q += DEC_THREADS) {  // whole 8-lane groups: nt is a multiple of 8
        const int blk = q >> 3, m = blk / KB, kb = blk - m * KB;
        const u32x2_t xv = kb * 32 < K ? *(const u32x2_t*)(xraw + (m * K + kb * 32) * 2 + (q & 7) * 8) : u32x2_t{0u, 0u};
        quantize_q8_1_x8(xv, q & 7, xq_lds + m * xq_row + kb * QB8_1, &xs_lds[blk]);  // blk == m * KB + kb
      }
    }
  };
  load_x(0, min(mch, nm));
  // the weight loads after the x pieces, every one issued (a lane past the row's units
  // re-reads its last unit), so that exactly NW vector memory instructions follow the x
  // pieces: x is quantised while the weights are still on their way
  __builtin_amdgcn_sched_barrier(0);
  typename U::W w[2][UPL];
#pragma unroll
  for (int j = 0; j < UPL; ++j) {
    const int uj = min(j0 + LPR * j, units - 1);
    U::load(wg, uj, grid, w[0][j]);
    U::load(wu, uj, grid, w[1][j]);
  }
  __builtin_amdgcn_sched_barrier(0);
  constexpr int NW = 2 * UPL * U::NLD;
  constexpr int NWC = NW < 63 ? NW : 63;
  __builtin_amdgcn_s_waitcnt((NWC & 15) | ((NWC >> 4) << 14) | (7 << 4) | (15 << 8));  // vmcnt(NWC): x has landed
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();  // every wave's x pieces (no workgroup fence: it would wait for the weights)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  quantize_x(min(mch, nm));
#pragma unroll
  for (int j = 0; j < UPL; ++j)
    if (j0 + LPR * j < units) {
      U::finish(w[0][j], grid);
      U::finish(w[1][j], grid);
    }
  for (int c0 = 0; c0 < nm; c0 += mch) {
    const int nc = min(mch, nm - c0);
    if (c0 > 0) {
      load_x(c0, nc);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      quantize_x(nc);
    }
    __syncthreads();
    for (int m = 0; m < nc; ++m) {
      float vg = 0.0f, vu = 0.0f;
#pragma unroll
      for (int j = 0; j < UPL; ++j) {
        const int u = j0 + LPR * j;
        if (u < units) {
          int ub0, ub1;
          U::qblocks(u, ub0, ub1);
          Act<U::NQ> a;
          load_act<U::NQ>(xq_lds + m * xq_row, ub0, ub1, a);
          // the int8 sums the units need, computed once per block in quantize_x
          if constexpr (needs_sums(TYPE)) act_sums<TYPE>(a, xs_lds[m * KB + ub0], xs_lds[m * KB + ub1]);
          vg += U::dot(w[0][j], a);
          vu += U::dot(w[1][j], a);
        }
      }
      vg = group_sum<LPR>(vg);
      vu = group_sum<LPR>(vu);
      if (j0 == 0) {  // the GEMV's bf16 outputs
        gu[m][i] = bf16_round(vg);
        gu[m][DEC_RG + i] = bf16_round(vu);
      }
    }
    __syncthreads();
    silu_h_q8_1(gu, nc, mem + c0, hq, hq_stride, g);
    __syncthreads();
  }
}

// One block per DEC_DR hidden rows. The hot routes are grouped by slot (counting sort in
// LDS) and, with STAGE, their q8_1 h rows copied into LDS in that order with one round of
// loads, issued together with the first round's weight loads. Wave w takes the slots with
// routes w, w + DEC_WAVES, ... (DEC_SPW per round), loads the block's rows of all of them
// into registers first, then runs every route of each past them. Y (bf16, the GEMV output
// dtype) stays in LDS; the block ends with the weighted top-k sum of its rows.
template <int TYPE, int LPR, bool STAGE>
__global__ __launch_bounds__(DEC_THREADS) void decode_down_combine(const uint8_t* __restrict__ hq, int64_t hq_stride,
                                                                   int K, int N, const int32_t* __restrict__ slot_ids,
                                                                   const float* __restrict__ topk_w, int T, int top_k,
                                                                   int S, const uint8_t* __restrict__ W2,
                                                                   int w_is_table, int64_t w_stride,
                                                                   __bf16* __restrict__ y) {
  using U = DUnit<TYPE>;
  constexpr int RPW = 64 / LPR;         // rows per wave pass
  constexpr int RIT = DEC_DR / RPW;     // passes over the block's rows
  // slots per wave and round (registers: SPW * RIT units; Q6_K's raw units are the largest)
  constexpr int SPW = (TYPE == GGML_Q6_K ? DEC_SPW / 2 : DEC_SPW) / RIT;
  static_assert(RIT >= 1 && DEC_DR % RPW == 0 && SPW >= 1, "row split");
  __shared__ __attribute__((aligned(16))) uint8_t hl[STAGE ? DEC_HL_LDS : 16];  // h rows, slot order
  __shared__ int cnt[DEC_MAX_SLOTS];   // routes per slot
  __shared__ int beg[DEC_MAX_SLOTS];   // first position of the slot's routes
  __shared__ int fill[DEC_MAX_SLOTS];  // next free position of the slot
  __shared__ int act_slots[DEC_MAX_SLOTS];
  __shared__ int order[DEC_MAX_ROUTES];   // hot routes grouped by slot
  __shared__ int pos_of[DEC_MAX_ROUTES];  // route -> index in order (-1: not hot)
  __shared__ float twl[DEC_MAX_ROUTES];
  __shared__ float yv[DEC_MAX_ROUTES][DEC_DR];
  // int8 half-block sums of the staged h blocks (the units' Unit::prep sums, once per block)
  __shared__ int2 hs_lds[STAGE && needs_sums(TYPE) ? DEC_HL_LDS / QB8_1 : 1];
  __shared__ int wsum[DEC_WAVES];
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int R = T * top_k;
  const int c0 = blockIdx.x * DEC_DR;
  // counting sort of the hot routes by slot (the order inside a slot is irrelevant: every
  // route's row sums are independent, and pos_of keeps each route's place)
  cnt[tid] = 0;  // DEC_MAX_SLOTS <= DEC_THREADS entries
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  const int sid = tid < R ? slot_ids[tid] : -1;
  if (tid < R) twl[tid] = topk_w[tid];
  const bool hot = sid >= 0 && sid < S;
  __syncthreads();
  if (hot) atomicAdd(&cnt[sid], 1);
  __syncthreads();
  // one scan gives each slot its start (low 16 bits) and its rank among the slots with
  // routes (high bits): counts are at most DEC_MAX_ROUTES, ranks at most DEC_MAX_SLOTS
  const int c = cnt[tid];
  int tot;
  const int packed = block_excl_scan(c | ((c > 0 ? 1 : 0) << 16), wsum, tot);
  beg[tid] = packed & 0xFFFF;
  fill[tid] = packed & 0xFFFF;
  if (c > 0) act_slots[packed >> 16] = tid;
  const int n_act = tot >> 16, n_hot = tot & 0xFFFF;
  __syncthreads();
  if (hot) {
    const int at = atomicAdd(&fill[sid], 1);
    order[at] = tid;
    pos_of[tid] = at;
  } else if (tid < R) {
    pos_of[tid] = -1;
  }
  __syncthreads();
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
    if constexpr (STAGE) {
      if (base == 0) {  // uniform; the h rows of every hot route, behind the first weight loads
        // buffer loads straight into LDS, 16 bytes a lane: piece q (16 bytes of the row of
        // position q / cpr) lands at hl + 16 q, one wave instruction per 64 pieces
        const int cpr = (int)(hq_stride / 16);
        const int nq = n_hot * cpr;
        const uint32_t hq_bytes = (uint32_t)(R * hq_stride);  // <= DEC_HL_LDS
        const __amdgpu_buffer_rsrc_t h_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)hq, (short)0, hq_bytes, 0x00020000);
        for (int q0 = wave * 64; q0 < nq; q0 += DEC_THREADS) {  // uniform per wave
          const int q = q0 + lane;
          // pieces past nq read past the buffer: zeros
          const uint32_t off = q < nq ? (uint32_t)(order[q / cpr] * hq_stride + (q % cpr) * 16) : hq_bytes;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(h_rsrc, (__attribute__((address_space(3))) void*)(hl + q0 * 16), 16,
                                                   (int)off, 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the pieces (and the weights) have landed
        __syncthreads();
        if constexpr (needs_sums(TYPE)) {
          const int nb = n_hot * (int)(hq_stride / QB8_1);
          for (int b = tid; b < nb; b += DEC_THREADS) {
            const uint32_t* qw = (const uint32_t*)(hl + b * QB8_1 + 4);
            int lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              lo = dot4(0x01010101u, qw[i], lo);
              hi = dot4(0x01010101u, qw[4 + i], hi);
            }
            hs_lds[b] = int2{lo, hi};
          }
          __syncthreads();
        }
      }
    }

#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (sl[j] < 0) continue;  // uniform per wave
      if (ulive)
#pragma unroll
        for (int r = 0; r < RIT; ++r) U::finish(w[j][r], grid);  // the others' loads stay in flight
      const int e = sl[j];
      const int b0 = beg[e], b1 = b0 + cnt[e];
      // RB routes at a time (the last ones repeated past the slot's end, their results
      // dropped): the activation reads and the dot chains of all of them overlap
      constexpr int RB = U::NQ == 1 ? 4 : 2;
      for (int at = b0; at < b1; at += RB) {
        Act<U::NQ> a[RB];
        if (ulive) {
#pragma unroll
          for (int m = 0; m < RB; ++m) {
            const int am = min(at + m, b1 - 1);
            if constexpr (STAGE) {
              load_act<U::NQ>(hl + am * (int)hq_stride, ub0, ub1, a[m]);
              if constexpr (needs_sums(TYPE)) {
                const int hb = am * (int)(hq_stride / QB8_1);
                act_sums<TYPE>(a[m], hs_lds[hb + ub0], hs_lds[hb + ub1]);
              }
            } else {
              load_act<U::NQ>(hq + (int64_t)order[am] * hq_stride, ub0, ub1, a[m]);
              U::prep(a[m]);
            }
          }
        }
#pragma unroll
        for (int r = 0; r < RIT; ++r) {
          float v[RB];
#pragma unroll
          for (int m = 0; m < RB; ++m) v[m] = ulive ? U::dot(w[j][r], a[m]) : 0.0f;
#pragma unroll
          for (int m = 0; m < RB; ++m) v[m] = group_sum<LPR>(v[m]);
#pragma unroll
          for (int m = 0; m < RB; ++m)
            if (u == 0 && at + m < b1) yv[at + m][r * RPW + lane / LPR] = bf16_round(v[m]);
        }
      }
    }
  }
  __syncthreads();
  // res[t, c] = bf16(sum over k ascending of bf16(Y[t,k,c] * bf16(w[t,k]))), eight k at a
  // time with every LDS read of the eight issued before the ordered sum
  for (int q = tid; q < T * DEC_DR; q += DEC_THREADS) {
    const int t = q / DEC_DR, i = q % DEC_DR;
    float acc = 0.0f;
    for (int k0 = 0; k0 < top_k; k0 += 8) {
      int atk[8];
      float wk[8], yk[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        atk[k] = k0 + k < top_k ? pos_of[t * top_k + k0 + k] : -1;
        wk[k] = k0 + k < top_k ? twl[t * top_k + k0 + k] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) yk[k] = atk[k] >= 0 ? yv[atk[k]][i] : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (atk[k] >= 0) acc += bf16_round(yk[k] * bf16_round(wk[k]));
    }
    y[(int64_t)t * K + c0 + i] = (__bf16)acc;
  }
}

template <int TYPE>
int launch_gate_up(const __bf16* x, const uint8_t* xq, int64_t K, int64_t N, const int32_t* slot_ids, int64_t top_k,
                   int64_t R, int64_t S, const uint8_t* W13, int w_is_table, int64_t w_stride, uint8_t* hq,
                   int64_t hq_stride, hipStream_t stream) {
  const int64_t xq_row = q8_1_row_bytes(K);
  const int64_t units = K / Unit<TYPE>::VALS;  // <= DEC_MAX_UNITS: decode_layer_fits
  const int upl = units <= DEC_GLPR ? 1 : units <= 2 * DEC_GLPR ? 2 : 4;
  int mch = (int)(DEC_MAX_XQ_LDS / xq_row < DEC_MCH_MAX ? DEC_MAX_XQ_LDS / xq_row : DEC_MCH_MAX);
  const int kb = (int)(q8_1_cols_padded(K) / 32);
  if (mch * kb > DEC_XQB) mch = DEC_XQB / kb;
  if (mch * K * 2 > DEC_XRAW_LDS) mch = (int)(DEC_XRAW_LDS / (K * 2));
  // the q8_1 rows of x arrive by 64-piece wave loads: room for one past the last row
  const size_t lds = (size_t)mch * (size_t)xq_row + (xq ? 1024 : 0);
  // one block per (slot, row group) walks all of the slot's routes: splitting them over more
  // blocks re-reads the weights once per extra block, which costs more than it saves at
  // decode sizes. Blocks past the slots with routes exit at once.
  const unsigned nb = (unsigned)(S * (N / DEC_RG));
#define KTMI_GU(P, Q)                                                                                         \
  decode_gate_up<TYPE, P, Q><<<nb, DEC_THREADS, lds, stream>>>(x, (int)K, (int)N, slot_ids, (int)top_k, (int)R, \
                                                                (int)S, W13, w_is_table, w_stride, hq, hq_stride, mch, xq)
  if (xq) {
    if (upl == 1) KTMI_GU(1, true);
    else if (upl == 2) KTMI_GU(2, true);
    else KTMI_GU(4, true);
  } else {
    if (upl == 1) KTMI_GU(1, false);
    else if (upl == 2) KTMI_GU(2, false);
    else KTMI_GU(4, false);
  }
#undef KTMI_GU
  static_assert(4 * DEC_GLPR >= DEC_MAX_UNITS, "units per lane");
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

template <int TYPE>
int launch_down(const uint8_t* hq, int64_t hq_stride, int64_t K, int64_t N, const int32_t* slot_ids,
                const float* topk_w, int64_t T, int64_t top_k, int64_t S, const uint8_t* W2, int w_is_table,
                int64_t w_stride, __bf16* y, hipStream_t stream) {
  const unsigned nb = (unsigned)(K / DEC_DR);
  // h rows staged in LDS when every route's row fits (hq_stride is a multiple of 576 bytes)
  const bool stage = T * top_k * hq_stride <= DEC_HL_LDS;
#define KTMI_DN(L, ST)                                                                                           \
  decode_down_combine<TYPE, L, ST><<<nb, DEC_THREADS, 0, stream>>>(hq, hq_stride, (int)K, (int)N, slot_ids, topk_w, \
                                                                  (int)T, (int)top_k, (int)S, W2, w_is_table,     \
                                                                  w_stride, y)
  switch (dec_lpr((int)(N / Unit<TYPE>::VALS))) {  // <= 16 units: decode_layer_fits
    case 16:
      if (stage) KTMI_DN(16, true); else KTMI_DN(16, false);
      break;
    default:
      if (stage) KTMI_DN(8, true); else KTMI_DN(8, false);
      break;
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

// workspace: q8_1(h) [R rows of N] | q8_1(x) [T rows of K] (used from DEC_PREQ_TOKENS tokens on)
int64_t decode_layer_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  auto al = [](int64_t v) { return (v + 255) & ~(int64_t)255; };
  return al(tokens * top_k * q8_1_row_bytes(L->inter)) + al(tokens * q8_1_row_bytes(L->hidden));
}

int launch_decode_layer(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                        int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots, R = tokens * top_k;
  const int64_t hq_stride = q8_1_row_bytes(N);
  const uint8_t* W13 = (const uint8_t*)L->w13;
  const uint8_t* W2 = (const uint8_t*)L->w2;
  const int64_t st13 = 2 * N * row_bytes(K, L->type13), st2 = K * row_bytes(N, L->type2);
  record_stage(0, stream);
  int rc;
  // x quantised once per token for the larger windows (the gate/up blocks of a slot would
  // each repeat it); below DEC_PREQ_TOKENS tokens the extra launch costs more than it saves
  uint8_t* xq = nullptr;
  if (tokens >= DEC_PREQ_TOKENS) {
    xq = ws + ((R * hq_stride + 255) & ~(int64_t)255);
    rc = launch_quantize_q8_1(x, KTMI_BF16, K, tokens, xq, stream);
    if (rc) return rc;
  }
  record_stage(1, stream);
  switch (L->type13) {
    case GGML_Q8_0: rc = launch_gate_up<GGML_Q8_0>((const __bf16*)x, xq, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_Q4_K: rc = launch_gate_up<GGML_Q4_K>((const __bf16*)x, xq, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_Q6_K: rc = launch_gate_up<GGML_Q6_K>((const __bf16*)x, xq, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
    case GGML_IQ3_S: rc = launch_gate_up<GGML_IQ3_S>((const __bf16*)x, xq, K, N, slot_ids, top_k, R, S, W13, L->w_is_table, st13, ws, hq_stride, stream); break;
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
