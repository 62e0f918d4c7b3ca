// Grouped hot-expert MoE for prefill chunks (gfx950: wave64, bf16 MFMA, 160 KB LDS).
//
//   1. sort_count / sort_scan / sort_scatter: a stable counting sort of the routes by
//      slot (ascending route index inside a slot, cold routes dropped). Each wave owns a
//      chunk of CHW consecutive routes; per-chunk histograms are scanned per slot, so
//      every route's position is a pure function of the ids: no host sync, no atomics
//      on positions, graph-capturable.
//   2. gemm<GATEUP>: for each (slot, tile of BM sorted routes, tile of N) the gathered
//      bf16 rows of x times the slot's gate and up rows, dequantised from raw GGUF blocks
//      into LDS (bf16, RNE of the exact fp32 dequant value), on
//      v_mfma_f32_32x32x16_bf16; the epilogue applies silu(gate)*up and writes bf16 rows
//      of H in sorted order.
//   3. gemm<down>: H rows (contiguous in sorted order) times the slot's down rows; the
//      epilogue scatters bf16 rows to Y in route order (p = t*top_k + k).
//   4. combine_routes: res[t] = sum over k ascending of bf16(Y[p] * bf16(w)), fp32, one
//      rounding (the reference's _combine order), skipping cold routes.
//
// Reference: the streamer's per-group dequant + cutlass_fused_moe + acc.add_ (P:40789-40819,
// dequant P:11471-11498), _combine (hot/kt_gguf_hot.py:43-71); the sort-by-expert follows the
// idea of moe_prepare_ids_kernel (P:31142-31162) with a deterministic stable order.
#include <type_traits>

#include "bpiece.h"
#include "kernels.h"

namespace ktmi {

namespace {

constexpr int CHW = 256;         // routes per wave chunk in the sort
constexpr int SORT_THREADS = 256;
constexpr int MAX_SLOTS = 512;

// tile configuration: 8 waves in 2 (M) x 4 (N), each 128 routes x 64 weight rows (8
// accumulators of 32 x 32, two waves per SIMD); tile = 256 routes x 256 weight rows
// (GATEUP: 128 gate + 128 up rows)
constexpr int BK = 64;
constexpr int FM = 4, FN = 2, WM = 2, WN = 4;
constexpr int NTHREADS = WM * WN * 64;
constexpr int NWAVES = WM * WN;
constexpr int BM = WM * FM * 32;   // routes per tile
constexpr int BNW = WN * FN * 32;  // weight rows per tile
constexpr int PIECES = 2 * BNW / NTHREADS;  // 32-value B pieces per thread per step
// LDS: the A tile in ADEPTH buffers (activations prefetched ADEPTH-1 steps ahead by direct
// global->LDS loads), the B tile (decoded weights) in 2 buffers; rows of 128 B in both,
// 16-byte slots swizzled (see lds_slot); 3 + 2 buffers fill the 160 KB of LDS, so the
// IQ3_S kernels (2 KB codebook in LDS) use 2 A buffers.
constexpr int A_BYTES = BM * BK * 2;
constexpr int B_BYTES = BNW * BK * 2;
constexpr int CPITCH_UP = BNW / 2 + 8;  // epilogue C tile pitches (bf16 elements)
constexpr int CPITCH_DN = BNW + 8;
constexpr int SMEM_C = BM * CPITCH_DN * 2;
template <int TYPE>
constexpr int adepth() { return TYPE == GGML_IQ3_S ? 2 : 3; }
template <int TYPE>
constexpr int smem_bytes() {
  return adepth<TYPE>() * A_BYTES + 2 * B_BYTES > SMEM_C ? adepth<TYPE>() * A_BYTES + 2 * B_BYTES : SMEM_C;
}
static_assert(3 * A_BYTES + 2 * B_BYTES <= 160 * 1024, "LDS");

// ---- route sort by slot. hist is slot-major: hist[e * nch + chunk].

__global__ __launch_bounds__(SORT_THREADS) void sort_count(const int32_t* __restrict__ slot_ids, int64_t R, int S,
                                                           int32_t* __restrict__ hist, int64_t nch) {
  __shared__ int cnt[SORT_THREADS / 64][MAX_SLOTS];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t ch = (int64_t)blockIdx.x * (SORT_THREADS / 64) + w;
  for (int e = lane; e < S; e += 64) cnt[w][e] = 0;
  __syncthreads();
  if (ch < nch) {
    const int64_t p0 = ch * CHW;
    for (int i = lane; i < CHW; i += 64) {
      const int64_t p = p0 + i;
      if (p < R) {
        const int e = slot_ids[p];
        if (e >= 0 && e < S) atomicAdd(&cnt[w][e], 1);
      }
    }
  }
  __syncthreads();
  if (ch < nch)
    for (int e = lane; e < S; e += 64) hist[(int64_t)e * nch + ch] = cnt[w][e];
}

// exclusive block scan of 256 ints in LDS (returns the total)
__device__ int block_scan_256(int* buf, int v) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int a = t >= off ? buf[t - off] : 0;
    __syncthreads();
    buf[t] += a;
    __syncthreads();
  }
  const int incl = buf[t];
  const int total = buf[255];
  __syncthreads();
  buf[t] = incl - v;
  return total;
}

// grid S: block e turns hist[e, :] into its exclusive prefix over chunks; tot[e] = total
__global__ __launch_bounds__(SORT_THREADS) void sort_scan_chunks(int32_t* __restrict__ hist, int64_t nch,
                                                                 int32_t* __restrict__ tot) {
  __shared__ int buf[SORT_THREADS];
  int32_t* h = hist + (int64_t)blockIdx.x * nch;
  const int64_t per = (nch + SORT_THREADS - 1) / SORT_THREADS;
  const int64_t c0 = threadIdx.x * per;
  int sum = 0;
  for (int64_t c = c0; c < c0 + per && c < nch; ++c) sum += h[c];
  const int total = block_scan_256(buf, sum);
  int run = buf[threadIdx.x];
  for (int64_t c = c0; c < c0 + per && c < nch; ++c) {
    const int v = h[c];
    h[c] = run;
    run += v;
  }
  if (threadIdx.x == 0) tot[blockIdx.x] = total;
}

// one block: seg[S+1] (route offsets) and tseg[S+1] (tile offsets, tiles of bm routes)
__global__ __launch_bounds__(SORT_THREADS) void sort_scan_slots(const int32_t* __restrict__ tot, int S,
                                                                int32_t* __restrict__ seg,
                                                                int32_t* __restrict__ tseg, int bm) {
  __shared__ int buf[SORT_THREADS];
  const int t = threadIdx.x;
  // two slots per thread (S <= 512)
  const int e0 = 2 * t, e1 = 2 * t + 1;
  const int a0 = e0 < S ? tot[e0] : 0, a1 = e1 < S ? tot[e1] : 0;
  const int b0 = (a0 + bm - 1) / bm, b1 = (a1 + bm - 1) / bm;
  const int ta = block_scan_256(buf, a0 + a1);
  const int ea = buf[t];
  const int tb = block_scan_256(buf, b0 + b1);
  const int eb = buf[t];
  if (e0 < S) { seg[e0] = ea; tseg[e0] = eb; }
  if (e1 < S) { seg[e1] = ea + a0; tseg[e1] = eb + b0; }
  if (t == 0) { seg[S] = ta; tseg[S] = tb; }
}

__global__ __launch_bounds__(SORT_THREADS) void sort_scatter(const int32_t* __restrict__ slot_ids, int64_t R, int S,
                                                             const int32_t* __restrict__ hist, int64_t nch,
                                                             const int32_t* __restrict__ seg,
                                                             int32_t* __restrict__ perm) {
  __shared__ int run[SORT_THREADS / 64][MAX_SLOTS];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t ch = (int64_t)blockIdx.x * (SORT_THREADS / 64) + w;
  if (ch >= nch) return;  // whole wave; no block-wide barrier below
  for (int e = lane; e < S; e += 64) run[w][e] = seg[e] + hist[(int64_t)e * nch + ch];
  __builtin_amdgcn_wave_barrier();
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t p0 = ch * CHW;
  for (int it = 0; it < CHW; it += 64) {
    const int64_t p = p0 + it + lane;
    int e = -1;
    if (p < R) {
      e = slot_ids[p];
      if (e >= S) e = -1;
    }
    const bool hot = e >= 0;
    // lanes holding the same slot id: intersect ballots over the id's bits
    uint64_t same = __ballot(hot);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(bit);
      same &= bit ? bb : ~bb;
    }
    int base = 0;
    if (hot) base = run[w][e];
    __builtin_amdgcn_wave_barrier();
    if (hot) {
      const int rank = __popcll(same & lt);
      perm[base + rank] = (int32_t)p;
      if ((same & lt) == 0) run[w][e] = base + __popcll(same);  // lowest lane of the group
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// GATEUP = true : A = x rows gathered through perm (token = p / top_k), Kdim = hidden,
//                 B rows = [gate n0..n0+BNW/2 ; up NI+n0..], out = H [R, NI] sorted rows.
// GATEUP = false: A = H rows m0.., Kdim = inter, B rows = down rows c0..c0+BNW,
//                 out = Y [routes, NI] at row perm[m] (NI = hidden).
//
// K loop over 64-value steps (bpiece.h maps step positions to row offsets), one barrier
// per step. Step k: load the raw B bytes of step k+2 into a register ring; MFMAs of step k
// from the A buffer k % AD and B buffer k & 1, with the decode of B(k+1) (raw bytes loaded
// a step earlier) into the other B buffer in the same basic block, so the scheduler can
// interleave the decode VALU with the matrix core, and the direct global->LDS loads of
// A(k+AD-1) spread over the sub-steps; wait for A(k+1) and the B stores; barrier.
// Loads past the last step re-read the last step (clamped, unused), keeping the loop
// branch-free.
// Workgroup barrier for the K loop. The caller has already waited for its own LDS writes
// (s_waitcnt): __syncthreads() would add a workgroup fence that also waits for every
// outstanding direct global->LDS load, including the ones meant to stay in flight. The
// wavefront-scope fences only keep the compiler from moving memory operations across.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A and B rows are 128 B in LDS; the 16-byte slot of chunk c of row r is
// c ^ (r & 7) ^ ((r >> 3) & 1): any 8 consecutive rows use 8 different slots (no conflict
// with 32 four-byte banks) and any 16 consecutive rows 16 different (row parity, slot)
// pairs (no conflict with 64 banks), for the 32-row MFMA operand reads.
__device__ __forceinline__ int lds_slot(int row, int chunk) { return chunk ^ (row & 7) ^ ((row >> 3) & 1); }

template <int TYPE, bool GATEUP>
__global__ __launch_bounds__(NTHREADS) void grouped_gemm(const uint16_t* __restrict__ A_src,
                                                         const int32_t* __restrict__ perm,
                                                         const int32_t* __restrict__ seg,
                                                         const int32_t* __restrict__ tseg, int S, int top_k,
                                                         const uint8_t* __restrict__ W, int w_is_table,
                                                         int64_t w_expert_stride, int64_t rb, int Kdim, int NI,
                                                         int NT, int64_t nblk, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[smem_bytes<TYPE>()];
  __shared__ uint32_t grid_lds[TYPE == GGML_IQ3_S ? 512 : 1];
  using BP = BPiece<TYPE>;

  // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin (pid % 8). All NT
  // N tiles of one M tile go to the same XCD, so they share its L2 for the gathered A
  // rows; M tiles rotate over the XCDs, so the real tiles (a prefix of the M range, the
  // rest exit at once) spread evenly. gridDim.x is a multiple of 8 * NT.
  const int64_t pid = blockIdx.x;
  const int64_t idx = pid >> 3;
  const int mt = (int)((idx / NT) * 8 + (pid & 7));
  const int nt = (int)(idx % NT);
  if ((int64_t)mt * NT + nt >= nblk) return;
  const int total_tiles = tseg[S];
  if (mt >= total_tiles) return;
  int lo = 0, hi = S;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (tseg[mid] <= mt) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int m0 = seg[e] + (mt - tseg[e]) * BM;
  const int valid = min(BM, seg[e + 1] - m0);

  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_grid(grid_lds);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W)[e] : W + (int64_t)e * w_expert_stride;
  constexpr int AD = adepth<TYPE>();
  uint8_t* Abuf0 = smem;
  uint8_t* Bbuf0 = smem + AD * A_BYTES;

  // ---- A sources: direct loads, instruction j of wave w fills rows 8*(NWAVES*j + w) + lane/8
  constexpr int AJ = BM / (8 * NWAVES);
  int a_off[AJ];  // element offset of this lane's 16-byte chunk, without the step base
#pragma unroll
  for (int j = 0; j < AJ; ++j) {
    const int row = 8 * (NWAVES * j + wave) + (lane >> 3);
    const int chunk = lds_slot(row, lane & 7);  // the slot map is an involution per row
    const int r = min(row, valid - 1);
    int src_row;
    if constexpr (GATEUP) src_row = perm[m0 + r] / top_k;
    else src_row = m0 + r;
    a_off[j] = src_row * Kdim + BP::coff(chunk);
  }
  auto issue_a = [&](int sb, auto subc, int buf, int j0 = 0, int j1 = AJ) {
    constexpr int SUB = decltype(subc)::value;
    const int kb = 256 * sb + BP::template ksub<SUB>();
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      uint8_t* dst = Abuf0 + buf * A_BYTES + (8 * (NWAVES * j + wave)) * (BK * 2);
      __builtin_amdgcn_global_load_lds(A_src + a_off[j] + kb, dst, 16, 0, 0);
    }
  };

  // ---- B source: piece p of thread t is half (q & 1) of weight row q >> 1, q = t * PIECES + p
  const uint8_t* b_row[PIECES];
  int b_j[PIECES], b_h[PIECES];
#pragma unroll
  for (int p = 0; p < PIECES; ++p) {
    const int q = tid * PIECES + p;
    b_j[p] = q >> 1;
    b_h[p] = q & 1;
    int64_t wr;
    if constexpr (GATEUP) {
      const int half = BNW / 2;
      const int n0 = nt * half;
      wr = b_j[p] < half ? (n0 + b_j[p]) : (NI + n0 + (b_j[p] - half));
    } else {
      wr = (int64_t)nt * BNW + b_j[p];
    }
    b_row[p] = wexp + wr * rb;
  }
  auto store_b = [&](const uint32_t* breg, int p, int buf) {
    uint8_t* bd = Bbuf0 + buf * B_BYTES + b_j[p] * (BK * 2);
    const int c0 = BP::off0(b_h[p]) / 8, c1 = BP::off1(b_h[p]) / 8;
    u32x4_t v0 = {breg[0], breg[1], breg[2], breg[3]};
    u32x4_t v1 = {breg[4], breg[5], breg[6], breg[7]};
    u32x4_t v2 = {breg[8], breg[9], breg[10], breg[11]};
    u32x4_t v3 = {breg[12], breg[13], breg[14], breg[15]};
    *(u32x4_t*)(bd + 16 * lds_slot(b_j[p], c0)) = v0;
    *(u32x4_t*)(bd + 16 * lds_slot(b_j[p], c0 + 1)) = v1;
    *(u32x4_t*)(bd + 16 * lds_slot(b_j[p], c1)) = v2;
    *(u32x4_t*)(bd + 16 * lds_slot(b_j[p], c1 + 1)) = v3;
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // raw ring: slot (k & 1) holds the bytes of step k (loaded two steps ahead)
  typename BP::Raw raw[2][PIECES];
  uint32_t breg[16];
  const int nsb = Kdim / 256;  // super-block columns, 4 steps each
  const int lsb = nsb - 1;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  if constexpr (TYPE == GGML_IQ3_S) __syncthreads();
  issue_a(0, S0{}, 0);
  if constexpr (AD == 3) issue_a(0, S1{}, 1);
#pragma unroll
  for (int p = 0; p < PIECES; ++p) {
    BP::template load<0>(b_row[p], 0, b_h[p], grid_lds, raw[0][p]);
    BP::template load<1>(b_row[p], 0, b_h[p], grid_lds, raw[1][p]);
  }
#pragma unroll
  for (int p = 0; p < PIECES; ++p) {
    BP::template decode<0>(raw[0][p], grid_lds, breg);
    store_b(breg, p, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // step SUB of super-block column sb (step k = 4 sb + SUB); the B buffer parity and the
  // raw ring slot are SUB & 1, the A buffer is k % AD (abuf). Loads beyond the last step
  // re-read the last column (in bounds, unused), so the body has no branches.
  int abuf = 0;
  auto step = [&](int sb, auto subc) {
    constexpr int SUB = decltype(subc)::value;
    constexpr int buf = SUB & 1;
    constexpr int SUB1 = (SUB + 1) & 3, SUB2 = (SUB + 2) & 3;
    constexpr int SUBA = (SUB + AD - 1) & 3;  // step k + AD - 1
    const int sb2 = SUB < 2 ? sb : min(sb + 1, lsb);
    const int sba = SUB + AD - 1 < 4 ? sb : min(sb + 1, lsb);
    // raw bytes of step k+2 replace those of step k (decoded one step ago), then the A
    // tile of step k+AD-1: the A loads are the newest VMEM, so the wait below can leave
    // just them in flight
#pragma unroll
    for (int p = 0; p < PIECES; ++p) BP::template load<SUB2>(b_row[p], sb2, b_h[p], grid_lds, raw[buf][p]);
    int anext = abuf + AD - 1;
    if (anext >= AD) anext -= AD;
    const uint8_t* Ab = Abuf0 + abuf * A_BYTES;
    const uint8_t* Bb = Bbuf0 + buf * B_BYTES;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      // the A loads of step k+AD-1 go out over the last three MFMA sub-steps: the waves
      // leave the barrier together, and one burst of every wave's loads would queue them
      // behind each other at the address unit
      if (kk >= 16) {
        constexpr int NPART = 3;
        const int part = kk / 16 - 1;
        __builtin_amdgcn_sched_barrier(0);
        issue_a(sba, std::integral_constant<int, SUBA>{}, anext, part * AJ / NPART, (part + 1) * AJ / NPART);
        __builtin_amdgcn_sched_barrier(0);
      }
      bf16x8_t af[FM], bfr[FN];
      const int chunk = (kk >> 3) + (lane >> 5);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * FM * 32 + i * 32 + (lane & 31);
        af[i] = *(const bf16x8_t*)(Ab + row * (BK * 2) + lds_slot(row, chunk) * 16);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        int brow;
        if constexpr (GATEUP) {
          brow = (j < FN / 2) ? (wn * (FN / 2) * 32 + j * 32) : (BNW / 2 + wn * (FN / 2) * 32 + (j - FN / 2) * 32);
        } else {
          brow = wn * FN * 32 + j * 32;
        }
        const int row = brow + (lane & 31);
        bfr[j] = *(const bf16x8_t*)(Bb + row * (BK * 2) + lds_slot(row, chunk) * 16);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      // the decode of the next step, spread over the MFMA sub-steps
      if ((kk / 16) % (4 / PIECES) == 0) {
        const int p = (kk / 16) / (4 / PIECES);
        BP::template decode<SUB1>(raw[buf ^ 1][p], grid_lds, breg);
        store_b(breg, p, buf ^ 1);
      }
    }
    // A(k+1) has landed once at most the newest AJ VMEM ops (the A loads of step k+2) are
    // outstanding (vmcnt field in bits 3:0 and 15:14; expcnt 7 and lgkmcnt 15 = no wait);
    // with AD == 2 everything must land
    if constexpr (AD == 3) {
      static_assert(AJ < 16, "vmcnt encoding");
      __builtin_amdgcn_s_waitcnt(AJ | (7 << 4) | (15 << 8));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this thread's B stores
    lds_barrier();
    abuf = abuf + 1 == AD ? 0 : abuf + 1;
  };
  for (int sb = 0; sb < nsb; ++sb) {
    step(sb, S0{});
    step(sb, S1{});
    step(sb, S2{});
    step(sb, S3{});
  }

  __builtin_amdgcn_s_waitcnt(0);  // the clamped prefetches of the last steps
  __syncthreads();

  // ---- epilogue through LDS. 32x32 accumulator layout: lane l, element r -> column l%32,
  // row 8*(r/4) + 4*(l/32) + r%4. The C tile is staged as bf16 in LDS, then written out
  // in 16-byte row chunks.
  uint16_t* cs = (uint16_t*)smem;
  const int col = lane & 31;
  if constexpr (GATEUP) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * FM * 32 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
#pragma unroll
        for (int j = 0; j < FN / 2; ++j)
          cs[ml * CPITCH_UP + wn * (FN / 2) * 32 + j * 32 + col] = f2bf(silu_mul(acc[i][j][r], acc[i][j + FN / 2][r]));
      }
    __syncthreads();
    constexpr int CW = BNW / 2 / 8;  // 16-byte chunks per row
    const int n0 = nt * (BNW / 2);
    for (int c = tid; c < BM * CW; c += NTHREADS) {
      const int ml = c / CW, q = c % CW;
      if (ml < valid)
        *(u32x4_t*)(out + (int64_t)(m0 + ml) * NI + n0 + 8 * q) = *(const u32x4_t*)(cs + ml * CPITCH_UP + 8 * q);
    }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ml = wm * FM * 32 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
#pragma unroll
        for (int j = 0; j < FN; ++j) cs[ml * CPITCH_DN + wn * FN * 32 + j * 32 + col] = f2bf(acc[i][j][r]);
      }
    __syncthreads();
    constexpr int CW = BNW / 8;
    for (int c = tid; c < BM * CW; c += NTHREADS) {
      const int ml = c / CW, q = c % CW;
      if (ml < valid) {
        const int64_t p = perm[m0 + ml];
        *(u32x4_t*)(out + p * NI + (int64_t)nt * BNW + 8 * q) = *(const u32x4_t*)(cs + ml * CPITCH_DN + 8 * q);
      }
    }
  }
}

// res[t, c] = bf16( sum_{k asc, slot_ids >= 0} fp32( bf16( Y[p, c] * bf16(w[p]) ) ) ), 8 columns
// per thread
__global__ __launch_bounds__(256) void combine_routes(const uint16_t* __restrict__ Y, const float* __restrict__ w,
                                                      const int32_t* __restrict__ slot_ids, int S, int top_k,
                                                      int64_t K, uint16_t* __restrict__ res) {
  const int64_t t = blockIdx.y;
  for (int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; c < K; c += (int64_t)gridDim.x * blockDim.x * 8) {
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      const int64_t p = t * top_k + k;
      const int e = slot_ids[p];
      if (e < 0 || e >= S) continue;
      const float wk = bf2f(f2bf(w[p]));
      const u32x4_t v = *(const u32x4_t*)(Y + p * K + c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[2 * i] += bf2f(f2bf(bf2f(v[i] & 0xFFFF) * wk));
        a[2 * i + 1] += bf2f(f2bf(bf2f(v[i] >> 16) * wk));
      }
    }
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2bf2(a[2 * i], a[2 * i + 1]);
    *(u32x4_t*)(res + t * K + c) = o;
  }
}

template <int TYPE, bool GATEUP>
void launch_gemm(dim3 grid, hipStream_t stream, const uint16_t* A_src, const int32_t* perm, const int32_t* seg,
                 const int32_t* tseg, int S, int top_k, const void* W, int w_is_table, int64_t w_expert_stride,
                 int64_t rb, int Kdim, int NI, int NT, int64_t nblk, uint16_t* out) {
  grouped_gemm<TYPE, GATEUP><<<grid, NTHREADS, 0, stream>>>(A_src, perm, seg, tseg, S, top_k, (const uint8_t*)W,
                                                             w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out);
}

template <bool GATEUP>
int dispatch_gemm(int type, dim3 grid, hipStream_t stream, const uint16_t* A_src, const int32_t* perm,
                  const int32_t* seg, const int32_t* tseg, int S, int top_k, const void* W, int w_is_table,
                  int64_t w_expert_stride, int64_t rb, int Kdim, int NI, int NT, int64_t nblk, uint16_t* out) {
  switch (type) {
    case GGML_Q8_0: launch_gemm<GGML_Q8_0, GATEUP>(grid, stream, A_src, perm, seg, tseg, S, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out); break;
    case GGML_Q4_K: launch_gemm<GGML_Q4_K, GATEUP>(grid, stream, A_src, perm, seg, tseg, S, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out); break;
    case GGML_Q6_K: launch_gemm<GGML_Q6_K, GATEUP>(grid, stream, A_src, perm, seg, tseg, S, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out); break;
    case GGML_IQ3_S: launch_gemm<GGML_IQ3_S, GATEUP>(grid, stream, A_src, perm, seg, tseg, S, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out); break;
    default: set_error("grouped GEMM: ggml type %d has no kernel", type); return KTMI_ETYPE;
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

GroupedPlan grouped_plan(int64_t tokens, int64_t top_k, int64_t n_slots, int64_t hidden, int64_t inter) {
  GroupedPlan P{};
  P.routes = tokens * top_k;
  P.n_slots = n_slots;
  const int64_t nch = (P.routes + CHW - 1) / CHW;
  P.max_tiles = (P.routes + BM - 1) / BM + n_slots;
  int64_t o = 0;
  P.off_counts = o; o = align256(o + ((nch > 0 ? nch : 1) * n_slots + n_slots) * 4);
  P.off_seg = o; o = align256(o + (n_slots + 1) * 4);
  P.off_tseg = o; o = align256(o + (n_slots + 1) * 4);
  P.off_perm = o; o = align256(o + P.routes * 4);
  P.off_h = o; o = align256(o + P.routes * inter * 2);
  P.off_y = o; o = align256(o + P.routes * hidden * 2);
  P.total = o;
  return P;
}

int launch_grouped_layer(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                         int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, const GroupedPlan& P,
                         hipStream_t stream) {
  const int64_t R = P.routes;
  const int S = (int)L->n_slots;
  const int64_t K = L->hidden, N = L->inter;
  KTMI_REQUIRE(S >= 1 && S <= MAX_SLOTS, KTMI_EINVAL, "grouped layer: n_slots %d outside [1, %d]", S, MAX_SLOTS);
  KTMI_REQUIRE(K % BNW == 0 && K % 256 == 0, KTMI_EINVAL, "grouped layer: hidden %lld not a multiple of %d",
               (long long)K, BNW > 256 ? BNW : 256);
  KTMI_REQUIRE(N % (BNW / 2) == 0 && N % 256 == 0, KTMI_EINVAL,
               "grouped layer: intermediate %lld not a multiple of 256", (long long)N);
  if (tokens == 0) return KTMI_OK;
  int32_t* hist = (int32_t*)(ws + P.off_counts);
  int32_t* seg = (int32_t*)(ws + P.off_seg);
  int32_t* tseg = (int32_t*)(ws + P.off_tseg);
  int32_t* perm = (int32_t*)(ws + P.off_perm);
  uint16_t* H = (uint16_t*)(ws + P.off_h);
  uint16_t* Y = (uint16_t*)(ws + P.off_y);
  const int64_t nch = (R + CHW - 1) / CHW;
  int32_t* tot = hist + nch * S;
  const unsigned sblocks = (unsigned)((nch + 3) / 4);
  record_stage(0, stream);
  sort_count<<<sblocks, SORT_THREADS, 0, stream>>>(slot_ids, R, S, hist, nch);
  sort_scan_chunks<<<S, SORT_THREADS, 0, stream>>>(hist, nch, tot);
  sort_scan_slots<<<1, SORT_THREADS, 0, stream>>>(tot, S, seg, tseg, BM);
  sort_scatter<<<sblocks, SORT_THREADS, 0, stream>>>(slot_ids, R, S, hist, nch, seg, perm);
  KTMI_HIP_TRY(hipGetLastError());
  record_stage(1, stream);
  const int64_t rb13 = row_bytes(K, L->type13), rb2 = row_bytes(N, L->type2);
  const int64_t st13 = 2 * N * rb13, st2 = K * rb2;
  const int NT1 = (int)(N / (BNW / 2));
  const int64_t nblk1 = P.max_tiles * NT1;
  dim3 g1((unsigned)((nblk1 + 8 * NT1 - 1) / (8 * NT1) * (8 * NT1)));
  int rc = dispatch_gemm<true>(L->type13, g1, stream, x, perm, seg, tseg, S, (int)top_k, L->w13, L->w_is_table,
                               st13, rb13, (int)K, (int)N, NT1, nblk1, H);
  if (rc) return rc;
  record_stage(2, stream);  // no mid stage on this path: SiLU*mul is in the gate/up epilogue
  record_stage(3, stream);
  const int NT2 = (int)(K / BNW);
  const int64_t nblk2 = P.max_tiles * NT2;
  dim3 g2((unsigned)((nblk2 + 8 * NT2 - 1) / (8 * NT2) * (8 * NT2)));
  rc = dispatch_gemm<false>(L->type2, g2, stream, H, perm, seg, tseg, S, (int)top_k, L->w2, L->w_is_table, st2, rb2,
                            (int)N, (int)K, NT2, nblk2, Y);
  if (rc) return rc;
  record_stage(4, stream);
  for (int64_t t0 = 0; t0 < tokens; t0 += 65535) {
    const int64_t nt = tokens - t0 < 65535 ? tokens - t0 : 65535;
    dim3 gc((unsigned)((K / 8 + 255) / 256), (unsigned)nt);
    combine_routes<<<gc, 256, 0, stream>>>(Y + t0 * top_k * K, topk_w + t0 * top_k, slot_ids + t0 * top_k, S,
                                           (int)top_k, K, y + t0 * K);
  }
  record_stage(5, stream);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

}  // namespace ktmi
