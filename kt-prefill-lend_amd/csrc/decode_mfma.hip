// Decode-sized hot-expert layer on the matrix cores (KTMI_MODE_DECODE): three launches for up
// to DM_MAX_ROUTES routes and DM_MAX_TOKENS tokens, the weights decoded from their GGUF
// blocks straight into v_mfma_f32_16x16x32_bf16 operands (bpiece.h: the exact dequantised
// values, one bf16 rounding, the values the grouped prefill kernels and the dequant entry
// point use), the routes of one slot as the MFMA's 16 columns.
//
//   dm_gate_up      block (k-th slot with routes, 16 intermediate rows): the block's 16 gate
//                   and 16 up rows staged in LDS by direct loads; the 4 waves split the
//                   hidden dimension, each lane decodes its share of the gate row and the up
//                   row it owns and multiplies them against the bf16 x rows of the slot's
//                   routes; the partial sums meet in LDS, h = bf16(silu(g) * u) (the grouped
//                   epilogue's) goes to h [R, N] of the routes.
//   dm_down         block (k-th slot with routes, 64 hidden rows): each wave stages 16 down
//                   rows of the slot in LDS by direct loads, runs them against the h rows of
//                   the slot's routes and writes each route's outputs, rounded to bf16 (the
//                   reference's per-route bf16 output), to yv [R, K].
//   dm_combine      the weighted top-k sum in k order (hot/kt_gguf_hot.py:43-71).
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
// own from the slot ids (ballots, and a 16-word slot bitmap ORed over the wave by DPP into
// scalar registers): no block barrier before the weight loads are issued.
#include <type_traits>

#include "bpiece.h"
#include "kernels.h"

namespace ktmi {

namespace {

constexpr int DM_WAVES = 4;                   // gate/up block: waves over the hidden dimension
constexpr int DM_THREADS = DM_WAVES * 64;
constexpr int DM_RT = 16;                     // intermediate rows per gate/up block
constexpr int DN_WAVES = 4;                   // down block: waves over the block's hidden rows
constexpr int DN_THREADS = DN_WAVES * 64;
constexpr int DN_ROWS = 16;                   // hidden rows per down wave (the MFMA's rows)
constexpr int DN_TILE = DN_WAVES * DN_ROWS;   // hidden rows per down block
constexpr int DN_WREG = DM_DOWN_WAVE_LDS;     // a wave's staged down rows
static_assert(DM_MAX_ROUTES <= 256, "four routes a lane; a route id fits a byte");

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

// OR of a 32-bit value over the wave, in scalar registers: DPP inside each row of 16 lanes
// (quad swaps, then the half-row and row mirrors), then the four rows' values read out
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_or(uint32_t v) {
  return v | (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  asm volatile("" : "+v"(v));  // a vector register: the compiler may otherwise feed DPP a scalar one
  v = dpp_or<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_or<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_or<0x141>(v);  // row_half_mirror
  v = dpp_or<0x140>(v);  // row_mirror
  return (uint32_t)(__builtin_amdgcn_readlane((int)v, 0) | __builtin_amdgcn_readlane((int)v, 16) |
                    __builtin_amdgcn_readlane((int)v, 32) | __builtin_amdgcn_readlane((int)v, 48));
}

// The slots with routes as 16 words of 32 slots (S <= 512), the same in every lane (scalar
// registers): each word is the OR over the wave of the lanes' own route bits.
struct SlotSet {
  static constexpr int NW = 16;
  uint32_t word[NW];
  int total;
  __device__ __forceinline__ void build(const WaveRoutes& wr, int S) {
    const int nw = (S + 31) >> 5;
    total = 0;
#pragma unroll
    for (int c = 0; c < NW; ++c) {
      word[c] = 0u;
      if (c < nw) {  // uniform
        uint32_t m = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          m |= wr.sid[i] >= 0 && (wr.sid[i] >> 5) == c ? 1u << (wr.sid[i] & 31) : 0u;
        word[c] = wave_or(m);
        total += __popc(word[c]);
      }
    }
  }
  // the k-th slot with routes in ascending order, -1 past the last (uniform over the wave)
  __device__ __forceinline__ int kth(int k) const {
    if (k >= total) return -1;
    int e = -1;
#pragma unroll
    for (int c = 0; c < NW; ++c) {
      const int n = __popc(word[c]);
      if (e < 0 && k < n) {  // uniform: the word holding it; its k lowest set bits cleared
        uint32_t v = word[c];
        for (int j = k; j > 0; --j) v &= v - 1u;
        e = 32 * c + __ffs(v) - 1;
      }
      k -= n;
    }
    return e;
  }
};

// The routes of slot e in ascending order at mem[0 .. m) (LDS private to the wave, a byte a
// route: route ids are below DM_MAX_ROUTES = 256); returns m. m <= tokens unless a token
// lists a slot twice; either way every route of the slot is listed.
__device__ __forceinline__ int slot_routes(const WaveRoutes& wr, int e, uint8_t* mem) {
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool hit = wr.sid[i] == e;
    const uint64_t b = __ballot(hit);
    const int at = base + __popcll(b & below);
    if (hit) mem[at] = (uint8_t)(64 * i + lane);
    base += __popcll(b);
  }
  wave_fence();
  return base;
}

// K offset inside a super-block column of the 8 values lane group (p, h) holds for MFMA j of
// double step S2 (the piece's values 8j..8j+7)
template <class BP, int S2>
__device__ __forceinline__ int kpos(int p, int h, int j) {
  const int q = j < 2 ? BP::off0(h) / 8 + j : BP::off1(h) / 8 + j - 2;
  return BP::template ksub_hp<S2>(p) + BP::coff(q);
}

// One block per (k-th slot with routes, 16 intermediate rows). The block's 16 gate rows and
// 16 up rows (two contiguous ranges of the slot tensor, 32 row_bytes(K) bytes) are moved into
// LDS by direct loads all issued at once, so the weights in flight cost no registers and
// three blocks share a CU; the 4 waves then take a quarter of the hidden dimension each,
// decode their share of the staged rows into MFMA operands and multiply them with the x rows
// of the slot's routes (loaded into registers behind the direct loads); the partial sums
// meet in LDS and h = bf16(silu(g) * u) goes to h [R, N] of the routes.
template <int TYPE>
__global__ __launch_bounds__(DM_THREADS) void dm_gate_up(const uint16_t* __restrict__ x, int K, int N,
                                                         const int32_t* __restrict__ slot_ids, int R, int S,
                                                         int top_k, const uint8_t* __restrict__ W13, int w_is_table,
                                                         int64_t w_stride, uint16_t* __restrict__ hbuf) {
  using BP = BPiece<TYPE>;
  // one LDS object (see the down kernel): staged rows, the waves' partial sums, their
  // scratch, the IQ3_S codebook
  constexpr int PART_OFF = DM_GU_LDS;
  constexpr int SCR_OFF = PART_OFF + DM_WAVES * 2 * 4 * 64 * 4;
  constexpr int GRID_OFF = SCR_OFF + DM_WAVES * DM_MAX_ROUTES;
  constexpr int LDS_BYTES = GRID_OFF + (TYPE == GGML_IQ3_S ? 2048 : 16);
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];
  float (*part)[2][4][64] = (float(*)[2][4][64])(smem + PART_OFF);  // [wave][tile: gate, up]
  uint8_t (*scratch)[DM_MAX_ROUTES] = (uint8_t(*)[DM_MAX_ROUTES])(smem + SCR_OFF);
  uint32_t* grid = (uint32_t*)(smem + GRID_OFF);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = N / DM_RT;
  const int kslot = blockIdx.x / G, rg = blockIdx.x - kslot * G;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_sel(grid);
  WaveRoutes wr;
  wr.load(slot_ids, R, S);
  SlotSet ss;
  ss.build(wr, S);
  const int e = ss.kth(kslot);
  if (e < 0) return;  // the same in every wave: past the slots with routes
  // the slot's routes and the first 16 routes' x offsets before the direct loads into LDS
  uint8_t* mem = scratch[wave];
  const int m = slot_routes(wr, e, mem);
  const int ncg = (m + 15) >> 4;  // 16-route column groups
  const int r = lane & 15, p = (lane >> 4) & 1, h = (lane >> 5) & 1;
  const uint32_t x_bytes = (uint32_t)(R / top_k) * (uint32_t)K * 2u;
  uint32_t xoff = r < m ? (uint32_t)(mem[r] / top_k) * (uint32_t)K * 2u : x_bytes;
  const int64_t rb = row_bytes(K, TYPE);
  const int range = DM_RT * (int)rb;  // bytes of 16 rows, a multiple of 16
  {
    // the gate range at smem, the up range at smem + range: 1 KB pieces over the waves, the
    // last piece of a range moved back to end at the range's end (its bytes written twice,
    // with the same values)
    const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W13)[e] : W13 + (int64_t)e * w_stride;
    const int npc = (range + 1023) >> 10;
    for (int q = wave; q < 2 * npc; q += DM_WAVES) {  // uniform per wave
      const int t = q >= npc, qi = q - t * npc;
      const int off = min(qi << 10, range - 1024);  // range >= 1024: decode_mfma_fits
      const uint8_t* src = wexp + ((int64_t)(t ? N : 0) + (int64_t)DM_RT * rg) * rb;
      const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (uint32_t)range, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (__attribute__((address_space(3))) void*)(smem + t * range + off), 16,
                                               off + 16 * lane, 0, 0, 0);
    }
  }
  const uint8_t* wrow[2] = {smem + r * (int)rb, smem + range + r * (int)rb};  // staged gate row r, up row r
  // activation operand: column c = 16 cg + r is the slot's c-th route (its token's x row);
  // columns past the routes read past the buffer, which returns zeros
  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, x_bytes, 0x00020000);
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
  f32x4_t acc[2][2];  // [tile: gate, up][two in turn, so back-to-back MFMAs do not wait for each other]
  // two super-block columns (sb, and sb + 1 when has1) of both tiles: every LDS read of the
  // four pieces first, then their decodes and MFMAs (one wave a SIMD at small T: the reads'
  // latency is paid once, not four times)
  bf16x8_t xa[2][4], xc[2][4];  // the x operands of the two columns
  auto compute2 = [&](int sb, bool has1) {
    typename BP::Head hd[2][2];
    typename BP::Raw raw[2][2][2];
    const int sbb = has1 ? sb + 1 : sb;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int sc = c2 ? sbb : sb;
        BP::template load_head<LMem>(wrow[t], sc, h, hd[c2][t]);
        BP::template load_hp<0, LMem>(wrow[t], sc, h, p, grid, raw[c2][t][0]);
        BP::template load_hp<1, LMem>(wrow[t], sc, h, p, grid, raw[c2][t][1]);
      }
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      if (c2 == 1 && !has1) break;  // uniform
      const bf16x8_t (&xb)[2][4] = c2 ? xc : xa;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint32_t a[16];
        BP::template decode_hp<0>(hd[c2][t], raw[c2][t][0], grid, p, a);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j & 1] = mfma16(words8(&a[4 * j]), xb[0][j], acc[t][j & 1]);
        BP::template decode_hp<1>(hd[c2][t], raw[c2][t][1], grid, p, a);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][j & 1] = mfma16(words8(&a[4 * j]), xb[1][j], acc[t][j & 1]);
      }
    }
  };
  // output (row rr, column c): lane 16 (rr / 4) + c of each wave holds it as element rr % 4;
  // 16 consecutive threads write one route's 16 values of h (32 bytes)
  const int c = threadIdx.x >> 4, rr = threadIdx.x & 15;
  const int ln = 16 * (rr >> 2) + c, i = rr & 3;
  // one pass per 16 routes of the slot (a second one only past 16 routes)
  for (int cg = 0; cg < ncg; ++cg) {
    if (cg > 0) xoff = 16 * cg + r < m ? (uint32_t)(mem[16 * cg + r] / top_k) * (uint32_t)K * 2u : x_bytes;
    acc[0][0] = acc[0][1] = acc[1][0] = acc[1][1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // the x operands of two super-block columns in flight (all of a wave's with K = 2048)
    auto xissue = [&](int sb, bf16x8_t (&xb)[2][4]) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 4; ++j) xb[s2][j] = xload(xoff, sb, kp[s2][j]);
    };
    if (sb0 < sb1) xissue(sb0, xa);
    if (sb0 + 1 < sb1) xissue(sb0 + 1, xc);
    if (cg == 0) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged rows (and the x operands)
      __syncthreads();                    // every wave's pieces; the IQ3_S codebook
    }
    for (int sb = sb0; sb < sb1; sb += 2) {
      compute2(sb, sb + 1 < sb1);
      if (sb + 2 < sb1) xissue(sb + 2, xa);
      if (sb + 3 < sb1) xissue(sb + 3, xc);
    }
    if (cg > 0) __syncthreads();  // the previous pass has read the partial sums
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) part[wave][t][q][lane] = acc[t][0][q] + acc[t][1][q];
    __syncthreads();
    const int col = 16 * cg + c;
    if (col < m) {
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int w = 0; w < DM_WAVES; ++w) {
        g += part[w][0][i][ln];
        u += part[w][1][i][ln];
      }
      hbuf[(int64_t)mem[col] * N + DM_RT * rg + rr] = f2bf(dm_silu_mul(g, u));
    }
  }
}

// One block per (k-th slot with routes, DN_TILE hidden rows); wave w takes the tile's rows
// 16 w .. 16 w + 15. A wave moves its 16 down rows of the slot (contiguous in the slot
// tensor) into its LDS region by direct loads, brings the h rows of the slot's routes into
// registers behind them (L2 hits: every block of the slot reads the same rows), decodes the
// rows into MFMA operands and writes each route's 16 outputs, rounded to bf16 (the
// reference's per-route bf16 output), to yv [R, K]. The weighted top-k sum is a launch of its
// own (dm_combine): inside this one, the blocks of a tile would have to order themselves
// through device-scope fences, which write back and invalidate the whole L2 of their XCD.
template <int TYPE>
__global__ __launch_bounds__(DN_THREADS) void dm_down(const uint16_t* __restrict__ hbuf, int K, int N,
                                                      const int32_t* __restrict__ slot_ids, int R, int S,
                                                      const uint8_t* __restrict__ W2, int w_is_table, int64_t w_stride,
                                                      uint16_t* __restrict__ yv) {
  using BP = BPiece<TYPE>;
  // one LDS object: per wave its staged rows, then the waves' route lists, the IQ3_S codebook
  constexpr int MEM_OFF = DN_WAVES * DN_WREG;
  constexpr int GRID_OFF = MEM_OFF + DN_WAVES * DM_MAX_ROUTES;
  constexpr int LDS_BYTES = GRID_OFF + (TYPE == GGML_IQ3_S ? 2048 : 16);
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];
  uint32_t* grid = (uint32_t*)(smem + GRID_OFF);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ntile = K / DN_TILE;
  const int kslot = blockIdx.x / ntile, tile = blockIdx.x - kslot * ntile;
  const int c0 = tile * DN_TILE;
  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_sel(grid);
  WaveRoutes wr;
  wr.load(slot_ids, R, S);
  SlotSet ss;
  ss.build(wr, S);
  const int e = ss.kth(kslot);
  if (e < 0) return;  // the same in every wave: past the slots with routes
  // the slot's routes and the first column group's h offsets before any direct load into
  // LDS: the compiler makes an LDS access after such loads wait for them
  uint8_t* mem = smem + MEM_OFF + DM_MAX_ROUTES * wave;
  const int m = slot_routes(wr, e, mem);
  const int ncg = (m + 15) >> 4;
  const int r = lane & 15, p = (lane >> 4) & 1, h = (lane >> 5) & 1;
  const uint32_t hrow = 2u * (uint32_t)N;
  const uint32_t h_bytes = (uint32_t)R * hrow;
  // column c = 16 cg + r of the operand is the slot's c-th route; past the routes the
  // offset lies past the buffer, whose loads return zeros
  uint32_t hoff = r < m ? (uint32_t)mem[r] * hrow : h_bytes;
  const int64_t rb = row_bytes(N, TYPE);
  const int wbytes = DN_ROWS * (int)rb;  // a multiple of 16, at most DN_WREG (decode_mfma_fits)
  const int rw0 = c0 + DN_ROWS * wave;
  uint8_t* const region = smem + wave * DN_WREG;
  {
    const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W2)[e] : W2 + (int64_t)e * w_stride;
    const __amdgpu_buffer_rsrc_t w_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(wexp + (int64_t)rw0 * rb), (short)0, (uint32_t)wbytes, 0x00020000);
    // 1 KB a wave instruction; the lanes past the end of the last piece stay idle
    for (int q0 = 0; q0 < wbytes; q0 += 1024)
      if (q0 + 16 * lane < wbytes)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (__attribute__((address_space(3))) void*)(region + q0), 16,
                                                 q0 + 16 * lane, 0, 0, 0);
  }
  const uint8_t* wrow = region + r * (int)rb;
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
  const int nsb = N / 256;
  f32x4_t acc[2];
  // one super-block column against the operands hb[S2][j]; two accumulators in turn, so
  // back-to-back MFMAs do not wait for each other
  auto compute = [&](int sb, const bf16x8_t (&hb)[2][4]) {
    typename BP::Head hd;
    typename BP::Raw raw[2];
    BP::template load_head<LMem>(wrow, sb, h, hd);
    BP::template load_hp<0, LMem>(wrow, sb, h, p, grid, raw[0]);
    BP::template load_hp<1, LMem>(wrow, sb, h, p, grid, raw[1]);
    uint32_t a[16];
    BP::template decode_hp<0>(hd, raw[0], grid, p, a);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j & 1] = mfma16(words8(&a[4 * j]), hb[0][j], acc[j & 1]);
    BP::template decode_hp<1>(hd, raw[1], grid, p, a);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j & 1] = mfma16(words8(&a[4 * j]), hb[1][j], acc[j & 1]);
  };
  for (int cg = 0; cg < ncg; ++cg) {
    if (cg > 0) hoff = 16 * cg + r < m ? (uint32_t)mem[16 * cg + r] * hrow : h_bytes;
    acc[0] = acc[1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8_t ha[2][4], hc[2][4];  // two super-block columns in flight
    auto hissue = [&](int sb, bf16x8_t (&hb)[2][4]) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int j = 0; j < 4; ++j) hb[s2][j] = hload(hoff, sb, kp[s2][j]);
    };
    hissue(0, ha);
    if (nsb > 1) hissue(1, hc);
    if (cg == 0) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged rows (and the h operands)
      wave_fence();
      if constexpr (TYPE == GGML_IQ3_S) __syncthreads();  // the codebook
    }
    for (int sb = 0; sb < nsb; sb += 2) {
      compute(sb, ha);
      if (sb + 2 < nsb) hissue(sb + 2, ha);
      if (sb + 1 < nsb) {
        compute(sb + 1, hc);
        if (sb + 3 < nsb) hissue(sb + 3, hc);
      }
    }
    // lane l holds rows 4 (l / 16) + i of column l % 16: four consecutive bf16 of yv
    const int col = 16 * cg + r;
    if (col < m) {
      const int rt = mem[col];
      const uint32_t lo = (uint32_t)f2bf(acc[0][0] + acc[1][0]) | ((uint32_t)f2bf(acc[0][1] + acc[1][1]) << 16);
      const uint32_t hi = (uint32_t)f2bf(acc[0][2] + acc[1][2]) | ((uint32_t)f2bf(acc[0][3] + acc[1][3]) << 16);
      *(uint2*)(yv + (int64_t)rt * K + rw0 + 4 * (lane >> 4)) = make_uint2(lo, hi);
    }
  }
}

// y[t, c] = bf16( sum over k ascending, hot routes only, of bf16(Y * bf16(w)) ): a thread per
// (token, eight hidden columns); the loads of eight routes are issued before their sums
__global__ __launch_bounds__(256) void dm_combine(const uint16_t* __restrict__ yv, const int32_t* __restrict__ slot_ids,
                                                  const float* __restrict__ topk_w, int T, int top_k, int S, int K,
                                                  uint16_t* __restrict__ y) {
  const int q = blockIdx.x * 256 + threadIdx.x;
  const int G = K / 8;
  if (q >= T * G) return;
  const int t = q / G, c = 8 * (q - t * G);
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < top_k; k0 += 8) {
    int sl[8];
    float w[8];
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int rt = t * top_k + min(k0 + u, top_k - 1);  // past top_k: a repeat, not summed
      sl[u] = slot_ids[rt];
      w[u] = topk_w[rt];
      v[u] = *(const uint4*)(yv + (int64_t)rt * K + c);  // every route's row lies in yv
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k0 + u >= top_k || sl[u] < 0 || sl[u] >= S) continue;  // cold or past top_k: its yv row is stale
      const float wb = bf2f(f2bf(w[u]));
      const uint32_t wd[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf2f(f2bf(bf2f((uint16_t)(wd[i] & 0xFFFFu)) * wb));
        acc[2 * i + 1] += bf2f(f2bf(bf2f((uint16_t)(wd[i] >> 16)) * wb));
      }
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (uint32_t)f2bf(acc[2 * i]) | ((uint32_t)f2bf(acc[2 * i + 1]) << 16);
  *(uint4*)(y + (int64_t)t * K + c) = make_uint4(o[0], o[1], o[2], o[3]);
}

template <int TYPE>
int launch_dm_gate_up(const ktmi_layer* L, const uint16_t* x, const int32_t* slot_ids, int64_t tokens, int64_t top_k,
                      uint16_t* hbuf, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots, R = tokens * top_k;
  const int64_t st13 = 2 * N * row_bytes(K, TYPE);
  // blocks numbered (k-th slot with routes, row group), row group fastest; the blocks past
  // the slots with routes exit at once
  const unsigned nb = (unsigned)(S < R ? S : R) * (unsigned)(N / DM_RT);
  dm_gate_up<TYPE><<<nb, DM_THREADS, 0, stream>>>(x, (int)K, (int)N, slot_ids, (int)R, (int)S, (int)top_k,
                                                  (const uint8_t*)L->w13, L->w_is_table, st13, hbuf);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

template <int TYPE>
int launch_dm_down(const ktmi_layer* L, const uint16_t* hbuf, const int32_t* slot_ids, const float* topk_w,
                   int64_t tokens, int64_t top_k, uint16_t* yv, uint16_t* y, hipStream_t stream) {
  const int64_t K = L->hidden, N = L->inter, S = L->n_slots, R = tokens * top_k;
  const int64_t st2 = K * row_bytes(N, TYPE);
  // blocks numbered (k-th slot with routes, hidden tile), tile fastest; the blocks past the
  // slots with routes exit at once
  const unsigned nb = (unsigned)(S < R ? S : R) * (unsigned)(K / DN_TILE);
  dm_down<TYPE><<<nb, DN_THREADS, 0, stream>>>(hbuf, (int)K, (int)N, slot_ids, (int)R, (int)S, (const uint8_t*)L->w2,
                                               L->w_is_table, st2, yv);
  KTMI_HIP_TRY(hipGetLastError());
  const unsigned nc = (unsigned)((tokens * (K / 8) + 255) / 256);
  dm_combine<<<nc, 256, 0, stream>>>(yv, slot_ids, topk_w, (int)tokens, (int)top_k, (int)S, (int)K, y);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

}  // namespace

bool decode_mfma_fits(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  if (L->hidden % 256 || L->inter % 256) return false;
  const int64_t range13 = DM_RT * row_bytes(L->hidden, L->type13);  // 16 gate (or up) rows
  const int64_t rows2 = DN_ROWS * row_bytes(L->inter, L->type2);    // a down wave's 16 rows
  return tokens * top_k <= DM_MAX_ROUTES && tokens <= DM_MAX_TOKENS && L->n_slots <= 512 &&
         L->hidden % DN_TILE == 0 && range13 >= 1024 && 2 * range13 <= DM_GU_LDS && rows2 <= DN_WREG;
}

namespace {
int64_t up256(int64_t v) { return (v + 255) & ~(int64_t)255; }
}  // namespace

// h [R, N] bf16, then yv [R, K] bf16 (the routes' down outputs)
int64_t decode_mfma_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  const int64_t R = tokens * top_k;
  return up256(R * L->inter * 2) + up256(R * L->hidden * 2);
}

int launch_decode_mfma(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                       int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream) {
  const int64_t R = tokens * top_k;
  uint16_t* hbuf = (uint16_t*)ws;
  uint16_t* yv = (uint16_t*)(ws + up256(R * L->inter * 2));
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
    case GGML_Q8_0: rc = launch_dm_down<GGML_Q8_0>(L, hbuf, slot_ids, topk_w, tokens, top_k, yv, y, stream); break;
    case GGML_Q4_K: rc = launch_dm_down<GGML_Q4_K>(L, hbuf, slot_ids, topk_w, tokens, top_k, yv, y, stream); break;
    case GGML_Q6_K: rc = launch_dm_down<GGML_Q6_K>(L, hbuf, slot_ids, topk_w, tokens, top_k, yv, y, stream); break;
    case GGML_IQ3_S: rc = launch_dm_down<GGML_IQ3_S>(L, hbuf, slot_ids, topk_w, tokens, top_k, yv, y, stream); break;
    default: set_error("decode layer: ggml type %d has no kernel", L->type2); return KTMI_ETYPE;
  }
  record_stage(4, stream);
  record_stage(5, stream);
  return rc;
}

}  // namespace ktmi
