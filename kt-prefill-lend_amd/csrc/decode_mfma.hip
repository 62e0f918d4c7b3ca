// Decode-sized hot-expert layer on the matrix cores (KTMI_MODE_DECODE): two launches for up
// to DM_MAX_ROUTES routes and DM_MAX_TOKENS tokens, the weights decoded from their GGUF
// blocks straight into v_mfma_f32_16x16x32_bf16 operands (bpiece.h: the exact dequantised
// values, one bf16 rounding, the values the grouped prefill kernels and the dequant entry
// point use), the routes of one slot as the MFMA's 16 columns.
//
//   dm_gate_up      block (k-th slot with routes, 16 intermediate rows): the 4 waves split
//                   the hidden dimension; each lane decodes the gate row and the up row it
//                   owns and multiplies them against the bf16 x rows of the slot's routes;
//                   the partial sums meet in LDS, h = bf16(silu(g) * u) (the grouped
//                   epilogue's) goes to h [R, N] of the routes.
//   dm_down_combine block (8 hidden rows): each wave stages the rows of its slots (every
//                   eighth slot with routes) in LDS with direct loads issued at once, runs
//                   them against the h rows of the slots' routes, rounds each route's output
//                   to bf16 (the reference's per-route bf16 output) in LDS; then the weighted
//                   top-k sum in k order (hot/kt_gguf_hot.py:43-71) of the block's rows.
//
// Lane map (16x16x32 operands): row or column l % 16, k-chunk g = l / 16 (8 values). Lane
// group g holds the piece of BPiece step SUB = 2 s + (g & 1), half g >> 1 of each 128-value
// double step s of a super-block column; MFMA j of the double step takes the piece's values
// 8j..8j+7. The activation operand of column c reads the same K positions of its row, so
// every lane pair of A and B refers to the same k. The K order inside a super-block is a
// permutation, which leaves every dot product unchanged.
//
// Against the GEMV mode (decode_layer.hip, the reference's int8 numerics): no q8_1
// quantisation of x or h, fp32 sums of bf16 products; the outputs stay within the layer's
// relative-L2 bar against the fp64 FFN. Per route the work is a fixed number of MFMAs, so
// a slot with 12 routes costs what a slot with one does.
//
// Membership (the k-th slot with routes, a slot's routes) is computed by every wave on its
// own from the slot ids (ballots and a 16-word bitmap in LDS private to the wave): no block
// barrier before the weight loads are issued.
#include <type_traits>

#include "bpiece.h"
#include "kernels.h"

namespace ktmi {

namespace {

constexpr int DM_WAVES = 4;                   // gate/up block: waves over the hidden dimension
constexpr int DM_THREADS = DM_WAVES * 64;
constexpr int DM_RI = 16;                     // intermediate rows per gate/up block
constexpr int DM_CG = DM_MAX_TOKENS / 16;     // 16-route column groups of a slot, at most
constexpr int DN_WAVES = 8;                   // down block: waves over the slots
constexpr int DN_THREADS = DN_WAVES * 64;
constexpr int DN_RH = 8;                      // hidden rows per down block (MFMA rows 8..15 repeat them)
constexpr int DN_WREG = DM_DOWN_WAVE_LDS;     // staged down rows per wave and round
static_assert(DM_MAX_ROUTES <= 256, "four routes a lane");
static_assert(DM_MAX_TOKENS % 16 == 0 && DN_THREADS >= DN_RH * DM_MAX_TOKENS, "combine: a thread per (token, row)");

__device__ __forceinline__ f32x4_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t words8(const uint32_t* w) {
  const u32x4_t v = {w[0], w[1], w[2], w[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

// silu(g) * u as the grouped gate/up epilogue computes it
__device__ __forceinline__ float dm_silu_mul(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

__device__ __forceinline__ void wave_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The call's routes, four a lane: route 64 i + lane has slot sid[i] (-1: no slot here).
struct WaveRoutes {
  int sid[4];
  __device__ __forceinline__ void load(const int32_t* __restrict__ slot_ids, int R, int S) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 64 * i + lane;
      const int s = r < R ? slot_ids[r] : -1;
      sid[i] = s >= 0 && s < S ? s : -1;
    }
  }
};

// The slots with routes as a bitmap of 16 words (S <= 512) in LDS private to the wave; lane
// w < 16 keeps word w and the number of slots with routes in words 0..w.
struct SlotSet {
  uint32_t word;
  int incl, total;
  __device__ __forceinline__ void build(const WaveRoutes& wr, uint32_t* bm) {
    const int lane = threadIdx.x & 63;
    if (lane < 16) bm[lane] = 0u;
    wave_fence();  // a wave's LDS operations run in order; the fences keep the compiler's order
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (wr.sid[i] >= 0) atomicOr(&bm[wr.sid[i] >> 5], 1u << (wr.sid[i] & 31));
    wave_fence();
    word = lane < 16 ? bm[lane] : 0u;
    incl = __popc(word);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    total = __shfl(incl, 15, 64);
  }
  // the k-th slot with routes in ascending order, -1 past the last (uniform over the wave)
  __device__ __forceinline__ int kth(int k) const {
    if (k >= total) return -1;
    const int lane = threadIdx.x & 63;
    const int before = incl - __popc(word);
    const bool here = lane < 16 && before <= k && k < incl;
    const int w = __ffsll((unsigned long long)__ballot(here)) - 1;
    int e = 0;
    if (here) {
      uint32_t v = word;
      for (int j = k - before; j > 0; --j) v &= v - 1u;
      e = 32 * lane + __ffs(v) - 1;
    }
    return __shfl(e, w, 64);
  }
};

// The routes of slot e in ascending order at mem[0 .. m) (LDS private to the wave); returns m.
// A slot holds one expert, which a token routes to at most once, so m <= tokens <=
// DM_MAX_TOKENS; routes past that (ids repeating a slot within a token) are not computed.
__device__ __forceinline__ int slot_routes(const WaveRoutes& wr, int e, int* mem) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool hit = wr.sid[i] == e;
    const uint64_t b = __ballot(hit);
    const int at = base + __popcll(b & below);
    if (hit && at < DM_MAX_TOKENS) mem[at] = 64 * i + lane;
    base += __popcll(b);
  }
  wave_fence();
  return base < DM_MAX_TOKENS ? base : DM_MAX_TOKENS;
}

// K offset inside a super-block column of the 8 values lane group (p, h) holds for MFMA j of
// double step S2 (the piece's values 8j..8j+7)
template <class BP, int S2>
__device__ __forceinline__ int kpos(int p, int h, int j) {
  const int q = j < 2 ? BP::off0(h) / 8 + j : BP::off1(h) / 8 + j - 2;
  return BP::template ksub_hp<S2>(p) + BP::coff(q);
}

template <int TYPE>
__global__ __launch_bounds__(DM_THREADS) void dm_gate_up(const uint16_t* __restrict__ x, int K, int N,
                                                         const int32_t* __restrict__ slot_ids, int R, int S,
                                                         int top_k, const uint8_t* __restrict__ W13, int w_is_table,
                                                         int64_t w_stride, uint16_t* __restrict__ hbuf) {
  using BP = BPiece<TYPE>;
  __shared__ float part[DM_WAVES][DM_CG][2][4][64];  // the waves' partial sums, [tile: gate, up]
  __shared__ int scratch[DM_WAVES][16 + DM_MAX_TOKENS];
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = N / DM_RI;
  const int kslot = blockIdx.x / G, rg = blockIdx.x - kslot * G;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  WaveRoutes wr;
  wr.load(slot_ids, R, S);
  SlotSet ss;
  ss.build(wr, (uint32_t*)scratch[wave]);
  const int e = ss.kth(kslot);
  if (e < 0) return;  // the same in every wave: past the slots with routes
  int* mem = scratch[wave] + 16;
  const int m = slot_routes(wr, e, mem);
  const int ncg = (m + 15) >> 4;  // <= DM_CG: at most DM_MAX_TOKENS tokens

  const int r = lane & 15, p = (lane >> 4) & 1, h = (lane >> 5) & 1;
  const int64_t rb = row_bytes(K, TYPE);
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W13)[e] : W13 + (int64_t)e * w_stride;
  const uint8_t* wrow[2] = {wexp + (int64_t)(DM_RI * rg + r) * rb, wexp + (int64_t)(N + DM_RI * rg + r) * rb};
  // activation operand: column c = 16 cg + r is the slot's c-th route (its token's x row);
  // columns past the routes read past the buffer, which returns zeros
  const uint32_t x_bytes = (uint32_t)(R / top_k) * (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, x_bytes, 0x00020000);
  uint32_t xoff[DM_CG];
#pragma unroll
  for (int cg = 0; cg < DM_CG; ++cg) {
    const int c = 16 * cg + r;
    xoff[cg] = c < m ? (uint32_t)(mem[c] / top_k) * (uint32_t)K * 2u : x_bytes;
  }
  int kp[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kp[0][j] = kpos<BP, 0>(p, h, j);
    kp[1][j] = kpos<BP, 1>(p, h, j);
  }
  auto xload = [&](uint32_t off, int sb, int k) {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off + 2u * (uint32_t)(256 * sb + k), 0, 0));
    return __builtin_bit_cast(bf16x8_t, v);
  };

  // this wave's super-block columns
  const int nsb = K / 256;
  const int per = (nsb + DM_WAVES - 1) / DM_WAVES;
  const int sb0 = wave * per, sb1 = min(nsb, sb0 + per);

  struct Stage {
    typename BP::Head hd[2];
    typename BP::Raw raw[2][2];
    bf16x8_t xb[2][4];
  };
  auto issue = [&](int sb, Stage& st) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      BP::load_head(wrow[t], sb, h, st.hd[t]);
      BP::template load_hp<0>(wrow[t], sb, h, p, grid, st.raw[t][0]);
      BP::template load_hp<1>(wrow[t], sb, h, p, grid, st.raw[t][1]);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) st.xb[s][j] = xload(xoff[0], sb, kp[s][j]);
  };

  f32x4_t acc[DM_CG][2];
#pragma unroll
  for (int cg = 0; cg < DM_CG; ++cg) acc[cg][0] = acc[cg][1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int sb, const Stage& st, auto s2c) {
    constexpr int S2 = decltype(s2c)::value;
    uint32_t a[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t) BP::template decode_hp<S2>(st.hd[t], st.raw[t][S2], grid, p, a[t]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0][0] = mfma16(words8(&a[0][4 * j]), st.xb[S2][j], acc[0][0]);
      acc[0][1] = mfma16(words8(&a[1][4 * j]), st.xb[S2][j], acc[0][1]);
    }
#pragma unroll
    for (int cg = 1; cg < DM_CG; ++cg) {
      if (cg < ncg) {  // uniform: slots with more than 16 routes
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8_t xb = xload(xoff[cg], sb, kp[S2][j]);
          acc[cg][0] = mfma16(words8(&a[0][4 * j]), xb, acc[cg][0]);
          acc[cg][1] = mfma16(words8(&a[1][4 * j]), xb, acc[cg][1]);
        }
      }
    }
  };

  using Z0 = std::integral_constant<int, 0>;
  using Z1 = std::integral_constant<int, 1>;
  // two stages in turn, the next super-block's loads issued before this one's MFMAs (with
  // K = 2048 a wave's two super-blocks are all in flight before the first MFMA)
  Stage sa, sbuf;
  if (sb0 < sb1) issue(sb0, sa);
  if constexpr (TYPE == GGML_IQ3_S) __syncthreads();  // the codebook
  for (int sb = sb0; sb < sb1; sb += 2) {
    if (sb + 1 < sb1) issue(sb + 1, sbuf);
    compute(sb, sa, Z0{});
    compute(sb, sa, Z1{});
    if (sb + 1 < sb1) {
      if (sb + 2 < sb1) issue(sb + 2, sa);
      compute(sb + 1, sbuf, Z0{});
      compute(sb + 1, sbuf, Z1{});
    }
  }

#pragma unroll
  for (int cg = 0; cg < DM_CG; ++cg)
    if (cg < ncg)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][cg][t][i][lane] = acc[cg][t][i];
  __syncthreads();
  // output (row rr, column c): lane 16 (rr / 4) + c of each wave holds it as element rr % 4;
  // 16 consecutive threads write one route's 16 values of h (32 bytes)
  const int c = threadIdx.x >> 4, rr = threadIdx.x & 15;
  const int ln = 16 * (rr >> 2) + c, i = rr & 3;
  for (int cg = 0; cg < ncg; ++cg) {
    const int col = 16 * cg + c;
    if (col < m) {
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int w = 0; w < DM_WAVES; ++w) {
        g += part[w][cg][0][i][ln];
        u += part[w][cg][1][i][ln];
      }
      hbuf[(int64_t)mem[col] * N + DM_RI * rg + rr] = f2bf(dm_silu_mul(g, u));
    }
  }
}

// One block per DN_RH hidden rows; NSB = N / 256 when it is small (0: any N, a loop). Wave w takes the slots with routes w, w + DN_WAVES, ...:
// per round, as many as its LDS region holds, their DN_RH rows (contiguous in the slot
// tensor) moved into LDS by direct loads all issued at once; then slot by slot, the h rows
// of the slot's routes (the next slot's issued before this one's MFMAs) against the decoded
// rows. Each route's output is rounded to bf16 into LDS; the block ends with the weighted
// top-k sum in k order.
template <int TYPE, int NSB>
__global__ __launch_bounds__(DN_THREADS) void dm_down_combine(const uint16_t* __restrict__ hbuf, int K, int N,
                                                              const int32_t* __restrict__ slot_ids,
                                                              const float* __restrict__ topk_w, int T, int top_k,
                                                              int S, const uint8_t* __restrict__ W2, int w_is_table,
                                                              int64_t w_stride, uint16_t* __restrict__ y) {
  using BP = BPiece<TYPE>;
  // one LDS object (with several, the compiler makes every LDS read wait for all direct
  // loads into LDS, including the h loads meant to stay in flight): per wave its staged
  // rows, then the routes' outputs, the waves' scratch, hot flags and route weights, the
  // IQ3_S codebook
  constexpr int YV_OFF = DN_WAVES * DN_WREG;
  constexpr int SCR_INTS = 16 + DM_MAX_TOKENS + 2 * (DN_WREG / 1024);  // bitmap, routes, row addresses
  constexpr int SCR_OFF = YV_OFF + DM_MAX_ROUTES * DN_RH * 4;
  constexpr int HOT_OFF = SCR_OFF + DN_WAVES * SCR_INTS * 4;
  constexpr int WTS_OFF = HOT_OFF + DM_MAX_ROUTES * 4;
  constexpr int GRID_OFF = WTS_OFF + DM_MAX_ROUTES * 4;
  constexpr int LDS_BYTES = GRID_OFF + (TYPE == GGML_IQ3_S ? 2048 : 16);
  static_assert(LDS_BYTES <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];
  float (*yv)[DN_RH] = (float(*)[DN_RH])(smem + YV_OFF);
  int (*scratch)[SCR_INTS] = (int(*)[SCR_INTS])(smem + SCR_OFF);
  int* hot = (int*)(smem + HOT_OFF);
  float* wts = (float*)(smem + WTS_OFF);
  uint32_t* grid = (uint32_t*)(smem + GRID_OFF);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int R = T * top_k;
  const int c0 = blockIdx.x * DN_RH;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid);
  if (threadIdx.x < R) {
    const int s = slot_ids[threadIdx.x];
    hot[threadIdx.x] = s >= 0 && s < S;
    wts[threadIdx.x] = topk_w[threadIdx.x];
  }
  WaveRoutes wr;
  wr.load(slot_ids, R, S);
  SlotSet ss;
  ss.build(wr, (uint32_t*)scratch[wave]);
  int* mem = scratch[wave] + 16;
  if constexpr (TYPE == GGML_IQ3_S) __syncthreads();  // the codebook

  // MFMA row r holds block row r % DN_RH: rows 8..15 repeat 0..7 and their outputs are unused
  const int r = lane & 15, p = (lane >> 4) & 1, h = (lane >> 5) & 1;
  const int64_t rb = row_bytes(N, TYPE);
  const int slot_bytes = DN_RH * (int)rb;
  const int slot_lds = (slot_bytes + 1023) & ~1023;  // whole 64-lane direct loads
  const int per_round = DN_WREG / slot_lds;          // >= 1: decode_mfma_fits
  const int nsb = N / 256;
  const uint32_t h_bytes = (uint32_t)R * (uint32_t)N * 2u;
  const __amdgpu_buffer_rsrc_t h_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)hbuf, (short)0, h_bytes, 0x00020000);
  int kp[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kp[0][j] = kpos<BP, 0>(p, h, j);
    kp[1][j] = kpos<BP, 1>(p, h, j);
  }
  auto hload = [&](uint32_t off, int sb, int k) {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(h_rsrc, off + 2u * (uint32_t)(256 * sb + k), 0, 0));
    return __builtin_bit_cast(bf16x8_t, v);
  };

  uint64_t* waddr = (uint64_t*)(scratch[wave] + 16 + DM_MAX_TOKENS);  // the round's row addresses
  for (int k0 = wave; k0 < ss.total; k0 += DN_WAVES * per_round) {
    // this round: the wave's slots k0, k0 + DN_WAVES, ... (per_round of them at most). Their
    // rows' addresses first (a slot table read is waited for before any direct load is
    // issued, so that no wait for it drains them), then every direct load at once.
    int nk = 0;
    for (int k = k0; k < ss.total && nk < per_round; k += DN_WAVES, ++nk) {
      const int e = ss.kth(k);
      const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W2)[e] : W2 + (int64_t)e * w_stride;
      if (lane == 0) waddr[nk] = (uint64_t)(uintptr_t)(wexp + (int64_t)c0 * rb);
    }
    wave_fence();
    for (int n = 0; n < nk; ++n) {
      const uint64_t a = waddr[n];  // the same in every lane: scalar registers for the resource
      const uint64_t au = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                          ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
      const __amdgpu_buffer_rsrc_t w_rsrc =
          __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)au, (short)0, (uint32_t)slot_bytes, 0x00020000);
      uint8_t* dst = smem + wave * DN_WREG + n * slot_lds;
      for (int q0 = 0; q0 < slot_bytes; q0 += 1024)  // pieces past the rows read zeros (within slot_lds)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (__attribute__((address_space(3))) void*)(dst + q0), 16,
                                                 q0 + 16 * lane, 0, 0, 0);
    }
    // the slots in turn; h of the next slot's routes is loaded before this one's MFMAs
    struct HOps { bf16x8_t v[2][4]; };
    auto hissue = [&](uint32_t off, int sb, HOps& o) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) o.v[s][j] = hload(off, sb, kp[s][j]);
    };
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's staged rows (the only loads so far)
    wave_fence();
    for (int n = 0; n < nk; ++n) {
      const int e = ss.kth(k0 + n * DN_WAVES);
      const int m = slot_routes(wr, e, mem);
      const uint8_t* wrow = smem + wave * DN_WREG + n * slot_lds + (r % DN_RH) * (int)rb;
      for (int cg = 0; cg * 16 < m; ++cg) {
        const int col = 16 * cg + r;
        const uint32_t hoff = col < m ? (uint32_t)mem[col] * (uint32_t)N * 2u : h_bytes;
        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        auto step = [&](int sb, const HOps& ho) {
          typename BP::Head hd;
          typename BP::Raw raw[2];
          uint32_t a[2][16];
          BP::template load_head<LMem>(wrow, sb, h, hd);
          BP::template load_hp<0, LMem>(wrow, sb, h, p, grid, raw[0]);
          BP::template load_hp<1, LMem>(wrow, sb, h, p, grid, raw[1]);
          BP::template decode_hp<0>(hd, raw[0], grid, p, a[0]);
          BP::template decode_hp<1>(hd, raw[1], grid, p, a[1]);
#pragma unroll
          for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mfma16(words8(&a[s][4 * j]), ho.v[s][j], acc);
        };
        if constexpr (NSB > 0) {
          // every h operand of the slot's columns issued at once, then the super-blocks in
          // turn (straight-line code: the compiler counts each wait)
          HOps ho[NSB];
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb) hissue(hoff, sb, ho[sb]);
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb) step(sb, ho[sb]);
        } else {
          for (int sb = 0; sb < nsb; ++sb) {
            HOps ho;
            hissue(hoff, sb, ho);
            step(sb, ho);
          }
        }
        // output rows 4 (lane / 16) + i (< DN_RH: lanes 0..31), column lane % 16
        if (lane < 2 * 16 && col < m) {
#pragma unroll
          for (int i = 0; i < 4; ++i) yv[mem[col]][4 * (lane >> 4) + i] = bf2f(f2bf(acc[i]));
        }
      }
      wave_fence();  // mem is rewritten for the next slot
    }
  }
  __syncthreads();
  // y[t, c0 + i] = bf16( sum over k ascending, hot routes only, of bf16(Y * bf16(w)) )
  for (int q = threadIdx.x; q < T * DN_RH; q += DN_THREADS) {
    const int t = q / DN_RH, i = q - t * DN_RH;
    float accy = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      const int rt = t * top_k + k;
      if (hot[rt]) accy += bf2f(f2bf(yv[rt][i] * bf2f(f2bf(wts[rt]))));
    }
    y[(int64_t)t * K + c0 + i] = f2bf(accy);
  }
}

template <int TYPE>
int launch_dm_gate_up(const ktmi_layer* L, const uint16_t* x, const int32_t* slot_ids, int64_t tokens, int64_t top_k,
                      uint16_t* hbuf, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots, R = tokens * top_k;
  const int64_t st13 = 2 * N * row_bytes(K, TYPE);
  // blocks numbered (k-th slot with routes, row group), row group fastest; the blocks past
  // the slots with routes exit at once
  const unsigned nb = (unsigned)(S < R ? S : R) * (unsigned)(N / DM_RI);
  dm_gate_up<TYPE><<<nb, DM_THREADS, 0, stream>>>(x, (int)K, (int)N, slot_ids, (int)R, (int)S, (int)top_k,
                                                  (const uint8_t*)L->w13, L->w_is_table, st13, hbuf);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

template <int TYPE>
int launch_dm_down(const ktmi_layer* L, const uint16_t* hbuf, const int32_t* slot_ids, const float* topk_w,
                   int64_t tokens, int64_t top_k, uint16_t* y, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots;
  const int64_t st2 = K * row_bytes(N, TYPE);
#define KTMI_DM_DOWN(NSB)                                                                                      \
  dm_down_combine<TYPE, NSB><<<(unsigned)(K / DN_RH), DN_THREADS, 0, stream>>>(                                   \
      hbuf, (int)K, (int)N, slot_ids, topk_w, (int)tokens, (int)top_k, (int)S, (const uint8_t*)L->w2, L->w_is_table, \
      st2, y)
  switch (N / 256) {
    case 1: KTMI_DM_DOWN(1); break;
    case 2: KTMI_DM_DOWN(2); break;
    case 3: KTMI_DM_DOWN(3); break;
    default: KTMI_DM_DOWN(0); break;
  }
#undef KTMI_DM_DOWN
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

}  // namespace

bool decode_mfma_fits(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  const int64_t rb2 = row_bytes(L->inter, L->type2);
  const int64_t slot_lds = (DN_RH * rb2 + 1023) & ~(int64_t)1023;
  return tokens * top_k <= DM_MAX_ROUTES && tokens <= DM_MAX_TOKENS && L->n_slots <= 512 && L->hidden % 256 == 0 &&
         L->inter % 256 == 0 && L->hidden % DN_RH == 0 && slot_lds <= DN_WREG &&
         (L->type2 != GGML_Q8_0 || L->inter % 256 == 0);
}

int64_t decode_mfma_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  return ((tokens * top_k * L->inter * 2) + 255) & ~(int64_t)255;  // h [R, N] bf16
}

int launch_decode_mfma(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                       int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream) {
  uint16_t* hbuf = (uint16_t*)ws;
  record_stage(0, stream);
  record_stage(1, stream);
  int rc;
  switch (L->type13) {
    case GGML_Q8_0: rc = launch_dm_gate_up<GGML_Q8_0>(L, x, slot_ids, tokens, top_k, hbuf, stream); break;
    case GGML_Q4_K: rc = launch_dm_gate_up<GGML_Q4_K>(L, x, slot_ids, tokens, top_k, hbuf, stream); break;
    case GGML_Q6_K: rc = launch_dm_gate_up<GGML_Q6_K>(L, x, slot_ids, tokens, top_k, hbuf, stream); break;
    case GGML_IQ3_S: rc = launch_dm_gate_up<GGML_IQ3_S>(L, x, slot_ids, tokens, top_k, hbuf, stream); break;
    default: set_error("decode layer: ggml type %d has no kernel", L->type13); return KTMI_ETYPE;
  }
  if (rc) return rc;
  record_stage(2, stream);
  record_stage(3, stream);
  switch (L->type2) {
    case GGML_Q8_0: rc = launch_dm_down<GGML_Q8_0>(L, hbuf, slot_ids, topk_w, tokens, top_k, y, stream); break;
    case GGML_Q4_K: rc = launch_dm_down<GGML_Q4_K>(L, hbuf, slot_ids, topk_w, tokens, top_k, y, stream); break;
    case GGML_Q6_K: rc = launch_dm_down<GGML_Q6_K>(L, hbuf, slot_ids, topk_w, tokens, top_k, y, stream); break;
    case GGML_IQ3_S: rc = launch_dm_down<GGML_IQ3_S>(L, hbuf, slot_ids, topk_w, tokens, top_k, y, stream); break;
    default: set_error("decode layer: ggml type %d has no kernel", L->type2); return KTMI_ETYPE;
  }
  record_stage(4, stream);
  record_stage(5, stream);
  return rc;
}

}  // namespace ktmi
