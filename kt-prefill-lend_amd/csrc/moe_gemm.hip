// Grouped hot-expert MoE for prefill chunks (gfx950: wave64, bf16 MFMA, 160 KB LDS).
//
//   1. sort_count / sort_scan_chunks / sort_scatter: a stable counting sort of the routes by
//      slot (ascending route index inside a slot, cold routes dropped). Each wave owns a
//      chunk of CHW consecutive routes; per-chunk histograms are scanned per slot, so
//      every route's position is a pure function of the ids: no host sync, no atomics
//      on positions, graph-capturable.
//   2. gemm<GATEUP>: for each (slot, tile of BM sorted routes, tile of N) the gathered
//      bf16 rows of x (staged in LDS by direct buffer->LDS loads) times the slot's gate and
//      up rows, which each lane dequantises from raw GGUF blocks straight into its MFMA
//      operand registers (bf16, RNE of the exact fp32 dequant value), on
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

// tile configuration: 4 waves (one per SIMD); wave w owns FI fragments of 32 weight rows
// and all FJ fragments of 32 routes of the tile: FI x FJ accumulators of 32 x 32 (256
// accumulation registers per lane at FJ = 8). Tile = BNW weight rows x BM routes (GATEUP:
// the wave's first FI/2 fragments are gate rows, the others the up rows of the same
// columns). The weights never touch LDS: each lane loads the raw GGUF bytes of its FI rows
// and decodes them straight into MFMA operand registers; LDS holds only the activation
// tile. FJ is a kernel parameter: 8 (256-route tiles) for long chunks, 4 (128 routes) when
// 256-route tiles would leave CUs idle (grouped_fj); a 256-route kernel runs a slot's last
// tile with the 128-route body when it holds at most 128 routes.
constexpr int BK = 64;
constexpr int WN = 4, WM = 1;          // waves over weight rows x waves over routes
constexpr int NWAVES = WN * WM;
constexpr int NTHREADS = NWAVES * 64;
constexpr int FI = 2;
constexpr int BNW = WN * FI * 32;      // weight rows per tile
constexpr int A_ROW = BK * 2;          // bytes of one activation row per K step
template <int FJ>
constexpr int tile_m() { return WM * FJ * 32; }  // routes per tile
// activation buffers: steps k .. k+AD-1 in flight (direct global->LDS loads AD-1 steps
// ahead); rows of 128 B, 16-byte slots swizzled (lds_slot)
constexpr int AD = 4;
static_assert(AD * tile_m<8>() * A_ROW + 2048 <= 160 * 1024, "LDS: activation buffers + IQ3_S codebook");

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

// exclusive scan over a block of 256 threads, one int each: buf[t] = the sum of the values of
// threads before t; returns the total. Each wave scans its 64 values with lane shifts, one
// barrier joins the 4 wave totals; ends with the block synchronised.
__device__ int block_scan_256(int* buf, int v) {
  __shared__ int wsum[SORT_THREADS / 64];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(inc, o, 64);
    if (lane >= o) inc += u;
  }
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int k = 0; k < SORT_THREADS / 64; ++k) {
    const int x = wsum[k];
    before += k < w ? x : 0;
    total += x;
  }
  buf[t] = before + inc - v;
  __syncthreads();  // wsum may be written again; buf complete
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

// The tile table: position p (npos of them, a multiple of 8) belongs to XCD p % 8, and XCD x
// takes the contiguous range of tiles [x per, (x + 1) per), per = ceil(tb / 8), so a slot's
// tiles (and weights) stay in one XCD's L2. Entry p = {slot, first sorted route, routes in the
// tile, 0}, or all zero for a position without a tile. segl / tsegl: the slots' first sorted
// route and first tile (S + 1 entries each); positions p0, p0 + pstride, ...
__device__ __forceinline__ void fill_tile_table(const int* segl, const int* tsegl, int S, int tb, int bm,
                                                int4* __restrict__ tile_info, int64_t npos, int64_t p0,
                                                int64_t pstride) {
  const int64_t per = ((int64_t)tb + 7) / 8;
  for (int64_t p = p0; p < npos; p += pstride) {
    const int64_t local = p >> 3, i = (p & 7) * per + local;
    int4 info = int4{0, 0, 0, 0};
    if (local < per && i < tb) {
      // the tile's slot is the last e with tsegl[e] <= i (binary search)
      int lo = 0, hi = S - 1;  // tsegl[lo] <= i < tsegl[hi + 1]
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tsegl[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      const int q = (int)i - tsegl[lo];
      const int n = segl[lo + 1] - segl[lo];
      info = int4{lo, segl[lo] + q * bm, min(bm, n - q * bm), 0};
    }
    tile_info[p] = info;
  }
}

// The slot ids of chunk ch's CHW routes, CHW / 64 a lane (-1: cold, or past the routes)
struct ChunkIds {
  int e[CHW / 64];
  __device__ __forceinline__ void load(const int32_t* __restrict__ slot_ids, int64_t R, int S, int64_t ch) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < CHW / 64; ++k) {
      const int64_t p = ch * CHW + 64 * k + lane;
      const int v = p < R ? slot_ids[p] : -1;
      e[k] = v < S ? v : -1;
    }
  }
};

// One wave scatters the CHW routes of chunk ch (their slot ids in ids): run[e] (LDS, the
// wave's own) holds the slot's next sorted position for this chunk (set by the caller); a
// route's position is run[e] plus its rank among the lanes of its 64-route round holding the
// same slot (ballots intersected over the slot id's bits), so the order inside a slot is the
// route order.
__device__ __forceinline__ void scatter_chunk(const ChunkIds& ids, int64_t ch, int* run, int top_k,
                                              int32_t* __restrict__ perm, int32_t* __restrict__ tok) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int k = 0; k < CHW / 64; ++k) {
    const int64_t p = ch * CHW + 64 * k + lane;
    const int e = ids.e[k];
    const bool hot = e >= 0;
    uint64_t same = __ballot(hot);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(bit);
      same &= bit ? bb : ~bb;
    }
    int base = 0;
    if (hot) base = run[e];
    __builtin_amdgcn_wave_barrier();
    if (hot) {
      const int rank = __popcll(same & lt);
      perm[base + rank] = (int32_t)p;
      tok[base + rank] = (int32_t)(p / top_k);  // the gate/up GEMM's gathered row
      if ((same & lt) == 0) run[e] = base + __popcll(same);  // lowest lane of the group
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// grid (nch + 3) / 4: wave w of block b scatters the routes of chunk 4b + w to perm (and their
// tokens, p / top_k, to tok: the gate/up GEMM's gathered rows, no division there). Every
// block first scans the S slot totals itself (S <= 512, two per thread) for the slots' first
// sorted positions and first tiles (tiles of bm routes); block 0 writes seg[S+1] (route
// offsets) and tseg[S+1] (tile offsets). The grid's threads then fill the tile table in the
// order the GEMMs' blocks read it: position p (npos = a multiple of 8 of them) belongs to
// XCD p % 8, and XCD x takes the contiguous range of tiles [x per, (x + 1) per), per =
// ceil(tiles / 8), so a slot's tiles (and weights) stay in one XCD's L2. Entry p = {slot,
// first sorted route, routes in the tile, 0}, or all zero for a position without a tile
// (a GEMM block reads its tile in one load; no separate launch for the slot scan).
__global__ __launch_bounds__(SORT_THREADS) void sort_scatter(const int32_t* __restrict__ slot_ids, int64_t R, int S,
                                                             const int32_t* __restrict__ hist, int64_t nch,
                                                             const int32_t* __restrict__ tot,
                                                             int32_t* __restrict__ seg, int32_t* __restrict__ tseg,
                                                             int4* __restrict__ tile_info, int64_t npos, int bm,
                                                             int top_k, int32_t* __restrict__ perm,
                                                             int32_t* __restrict__ tok) {
  __shared__ int run[SORT_THREADS / 64][MAX_SLOTS];
  __shared__ int segl[MAX_SLOTS + 1];
  __shared__ int tsegl[MAX_SLOTS + 1];
  __shared__ int buf[SORT_THREADS];
  const int t = threadIdx.x;
  const int e0 = 2 * t, e1 = 2 * t + 1;
  const int a0 = e0 < S ? tot[e0] : 0, a1 = e1 < S ? tot[e1] : 0;
  const int b0 = (a0 + bm - 1) / bm, b1 = (a1 + bm - 1) / bm;
  const int ta = block_scan_256(buf, a0 + a1);
  const int ea = buf[t];
  const int tb = block_scan_256(buf, b0 + b1);
  const int eb = buf[t];
  if (e0 < S) { segl[e0] = ea; tsegl[e0] = eb; }
  if (e1 < S) { segl[e1] = ea + a0; tsegl[e1] = eb + b0; }
  if (t == 0) { segl[S] = ta; tsegl[S] = tb; }
  if (blockIdx.x == 0) {
    if (e0 < S) { seg[e0] = ea; tseg[e0] = eb; }
    if (e1 < S) { seg[e1] = ea + a0; tseg[e1] = eb + b0; }
    if (t == 0) { seg[S] = ta; tseg[S] = tb; }
  }
  __syncthreads();  // segl, tsegl
  fill_tile_table(segl, tsegl, S, tb, bm, tile_info, npos, (int64_t)blockIdx.x * SORT_THREADS + t,
                  (int64_t)gridDim.x * SORT_THREADS);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t ch = (int64_t)blockIdx.x * (SORT_THREADS / 64) + w;
  if (ch >= nch) return;  // whole wave; no block-wide barrier below
  ChunkIds ids;
  ids.load(slot_ids, R, S, ch);
  for (int e = lane; e < S; e += 64) run[w][e] = segl[e] + hist[(int64_t)e * nch + ch];
  __builtin_amdgcn_wave_barrier();
  scatter_chunk(ids, ch, run[w], top_k, perm, tok);
}

// Exclusive prefix sum over the SMALL_THREADS threads of a block (one value each); every
// thread gets the total too. wsum holds SMALL_WAVES ints; ends with the block synchronised.
constexpr int SMALL_THREADS = 1024;
constexpr int SMALL_WAVES = SMALL_THREADS / 64;
// chunks per wave of the one-block sort: one (4096 routes). Its scattered perm / tok stores all
// go through one CU's address unit, so beyond that the three-launch sort, whose stores spread
// over the CUs, is faster (2048 tokens x top-8 with four chunks a wave: 151 -> 164 us a layer;
// 512 tokens x top-8, one chunk a wave: 82.0 -> 80.3 us)
constexpr int SMALL_CPW = 1;
__device__ __forceinline__ int block_scan_1024(int* wsum, int v, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(inc, o, 64);
    if (lane >= o) inc += u;
  }
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < SMALL_WAVES; ++k) {
    const int x = wsum[k];
    before += k < w ? x : 0;
    total += x;
  }
  __syncthreads();  // wsum may be written again
  return before + inc - v;
}

// The whole route sort of a short chunk in one block, one launch instead of three: the
// outputs of sort_count + sort_scan_chunks + sort_scatter (perm, tok, seg, tseg, the tile
// table), the same values. Chunk c (CHW routes) is counted and scattered by wave
// c % SMALL_WAVES; the per-chunk counts (slot-major, then turned into each slot's prefix over
// the chunks) and the waves' running positions live in dynamic LDS: (nch + SMALL_WAVES) x S
// ints (sort_small_fits).
__global__ __launch_bounds__(SMALL_THREADS) void sort_small(const int32_t* __restrict__ slot_ids, int R, int S,
                                                            int nch, int32_t* __restrict__ seg,
                                                            int32_t* __restrict__ tseg, int4* __restrict__ tile_info,
                                                            int64_t npos, int bm, int top_k, int32_t* __restrict__ perm,
                                                            int32_t* __restrict__ tok) {
  extern __shared__ int dyn[];
  int* const hist = dyn;              // [S][nch]
  int* const run = dyn + S * nch;     // [SMALL_WAVES][S]
  __shared__ int segl[MAX_SLOTS + 1];
  __shared__ int tsegl[MAX_SLOTS + 1];
  __shared__ int tot_l[MAX_SLOTS];
  __shared__ int wsum[SMALL_WAVES];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  for (int i = t; i < S * nch; i += SMALL_THREADS) hist[i] = 0;
  // the wave's chunks w, w + SMALL_WAVES, ... (at most SMALL_CPW): their slot ids in registers
  ChunkIds ids[SMALL_CPW];
#pragma unroll
  for (int c = 0; c < SMALL_CPW; ++c) ids[c].load(slot_ids, R, S, w + (int64_t)SMALL_WAVES * c);
  __syncthreads();
#pragma unroll
  for (int c = 0; c < SMALL_CPW; ++c) {
    const int ch = w + SMALL_WAVES * c;
#pragma unroll
    for (int k = 0; k < CHW / 64; ++k)
      if (ids[c].e[k] >= 0) atomicAdd(&hist[ids[c].e[k] * nch + ch], 1);  // past the routes: -1
  }
  __syncthreads();
  // slot e's routes' prefix over its chunks (nch <= 64: lane ch of wave e % SMALL_WAVES), its
  // total in tot_l[e]
  for (int e = w; e < S; e += SMALL_WAVES) {
    const int v = lane < nch ? hist[e * nch + lane] : 0;
    int inc = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(inc, o, 64);
      if (lane >= o) inc += u;
    }
    if (lane < nch) hist[e * nch + lane] = inc - v;
    if (lane == 63) tot_l[e] = inc;
  }
  __syncthreads();
  const int a = t < S ? tot_l[t] : 0;
  int ta, tb;
  const int ea = block_scan_1024(wsum, a, ta);
  const int eb = block_scan_1024(wsum, (a + bm - 1) / bm, tb);
  if (t < S) {
    segl[t] = seg[t] = ea;
    tsegl[t] = tseg[t] = eb;
  }
  if (t == 0) {
    segl[S] = seg[S] = ta;
    tsegl[S] = tseg[S] = tb;
  }
  __syncthreads();  // segl, tsegl; the chunk prefixes
  fill_tile_table(segl, tsegl, S, tb, bm, tile_info, npos, t, SMALL_THREADS);
  int* const rw = run + w * S;
#pragma unroll
  for (int c = 0; c < SMALL_CPW; ++c) {
    const int ch = w + SMALL_WAVES * c;
    if (ch >= nch) break;  // uniform per wave
    for (int e = lane; e < S; e += 64) rw[e] = segl[e] + hist[e * nch + ch];
    __builtin_amdgcn_wave_barrier();
    scatter_chunk(ids[c], ch, rw, top_k, perm, tok);
  }
}

// routes up to which the one-block sort runs
constexpr int64_t SMALL_ROUTES = (int64_t)SMALL_WAVES * SMALL_CPW * CHW;
constexpr int SMALL_LDS = 60 * 1024;
bool sort_small_fits(int64_t R, int64_t S) {
  const int64_t nch = (R + CHW - 1) / CHW;
  static_assert(SMALL_ROUTES / CHW <= 64, "one lane per chunk in the chunk scan");
  return R <= SMALL_ROUTES && (nch + SMALL_WAVES) * S * 4 <= SMALL_LDS;
}

// silu(g) * u with the hardware reciprocal (1 ulp) in place of a division: the gate/up epilogue
// runs it 128 times a lane with no MFMA work left to hide it behind
__device__ __forceinline__ float silu_mul(float g, float u) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u; }

// Workgroup barrier for the K loop. The caller has already waited for its own LDS traffic:
// __syncthreads() would add a workgroup fence that also waits for every outstanding direct
// global->LDS load, including the ones meant to stay in flight. The wavefront-scope fences
// only keep the compiler from moving memory operations across.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt operand that waits until at most n vector memory operations are outstanding
// (vmcnt bits 3:0 and 15:14; expcnt 7 and lgkmcnt 15 mean no wait on those counters)
constexpr int wait_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Activation rows are 128 B in LDS; the 16-byte slot of chunk c of row r is
// c ^ (r & 7) ^ ((r >> 3) & 1): any 8 consecutive rows use 8 different slots and any 16
// consecutive rows 16 different (row parity, slot) pairs, so the 32-row MFMA operand reads
// are free of bank conflicts.
__device__ __forceinline__ int lds_slot(int row, int chunk) { return chunk ^ (row & 7) ^ ((row >> 3) & 1); }

// 128-route tiles of the light decodes (Q8_0, Q4_K) fit two waves per SIMD (accumulators in
// VGPRs, 256 registers a lane), so two blocks share a CU; Q6_K and IQ3_S would spill there.
template <int TYPE, int FJ>
constexpr int gemm_waves_per_simd() { return FJ == 8 || TYPE == GGML_Q6_K || TYPE == GGML_IQ3_S ? 1 : 2; }

// GATEUP = true : activations = x rows gathered through perm (here the sorted routes' tokens),
//                 Kdim = hidden, weight rows = [gate n0.. ; up NI+n0..], out = H [R, NI]
//                 sorted rows, silu(gate) * up.
// GATEUP = false: activations = H rows m0.., Kdim = inter, weight rows = down rows of the
//                 tile's columns, out = Y [routes, NI] at row perm[m] (NI = hidden).
//
// MFMA operands: srcA = weights (row = lane % 32 of a 32-row fragment), srcB = activations
// (column = route lane % 32); k = 8 (lane / 32) + [0, 8) of each 16-value sub-step. The
// K positions a lane covers in a 64-value step are those of its decoded piece (bpiece.h:
// half h = lane / 32 of the step, 16 values at off0(h) and 16 at off1(h)); sub-step s
// takes the piece's values 8s..8s+7, and reads the activation chunk at the same positions.
//
// K loop, step k (one barrier per step): raw weight bytes of step k+2 into a register ring
// (and, once per super-block column, the next column's scales into head_nxt); 4 sub-steps
// of FI x FJ MFMAs on the weights decoded one step earlier and the activation buffer
// k % AD, with the decode of step k+1 and the direct loads of activation step k+AD-1
// spread over the sub-steps (step 0 also issues steps 1 and 2: the prologue loads only
// step 0's activations and the first two steps' raw bytes). Loads past the last step
// re-read the last one (clamped, unused), keeping the loop branch-free.
//
// Epilogue: the accumulators are converted (GATEUP: silu(gate) * up) to bf16 and written
// out as row segments (the down GEMM's rows scatter to Y[perm[m]], whose indices are put in
// LDS right after the prologue): at 256-route tiles through a staging area of each wave's own, at
// 128-route tiles through a C tile in LDS over the activation buffers.
// LDS of one tile (one object: the IQ3_S codebook, the activation buffers, the down tile's
// output row indices, the per-wave staging areas of 256-route tiles)
template <int TYPE, bool GATEUP, int FJ>
constexpr int gemm_lds_bytes() {
  constexpr int STG_COLS = GATEUP ? FI / 2 * 32 : FI * 32;
  return (TYPE == GGML_IQ3_S ? 512 * 4 : 0) + AD * tile_m<FJ>() * A_ROW + (GATEUP ? 0 : tile_m<FJ>() * 4) +
         (FJ == 8 ? NWAVES * 32 * STG_COLS * 2 : 0);
}

// One tile: routes m0 .. m0 + valid - 1 of the slot whose weights start at wexp, weight-row
// tile nt. smem holds at least gemm_lds_bytes<TYPE, GATEUP, FJ>() and, for IQ3_S, the staged
// codebook at offset 0 (visible after the prologue's barrier).
template <int TYPE, bool GATEUP, int FJ>
__device__ __forceinline__ void gemm_tile(uint8_t* smem, const uint16_t* __restrict__ A_src, uint32_t a_bytes,
                                          const int32_t* __restrict__ perm, int top_k,
                                          const uint8_t* __restrict__ wexp, int64_t rb, int Kdim, int NI, int nt,
                                          int m0, int valid, uint16_t* __restrict__ out, uint32_t out_bytes) {
  constexpr int BM = tile_m<FJ>();
  constexpr int A_BYTES = BM * A_ROW;
  constexpr int AJ = A_BYTES / (16 * NTHREADS);  // direct loads per thread per step
  static_assert(AJ % 2 == 0, "A loads are spread over the 2 regions of a step");
  // one LDS object: the IQ3_S codebook, then the activation buffers. With a second
  // __shared__ variable the compiler tracks the direct buffer->LDS loads per object and
  // waits for all of them (vmcnt(0)) before every LDS read, which drains the prefetch. The
  // codebook's offset 0 lets each lookup take its address straight from the index (no add).
  constexpr int GRID_BYTES = TYPE == GGML_IQ3_S ? 512 * 4 : 0;
  constexpr int OROW_BYTES = GATEUP ? 0 : BM * 4;  // down: the tile's output row indices
  // 256-route tiles (one block per CU, LDS to spare): each wave stages its own 32-route slices
  // of the C tile, so the epilogue needs no workgroup barrier
  constexpr bool WAVE_STG = FJ == 8;
  constexpr int STG_COLS = GATEUP ? FI / 2 * 32 : FI * 32;  // the wave's output columns
  constexpr int STG_WAVE = 32 * STG_COLS * 2;                // 32 routes of them, bf16
  uint32_t* const grid_lds = (uint32_t*)smem;
  uint8_t* const a_lds = smem + GRID_BYTES;  // activation buffer b at a_lds + b * A_BYTES
  int32_t* const orow_lds = (int32_t*)(a_lds + AD * A_BYTES);
  using BP = BPiece<TYPE>;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  const int h = lane >> 5, l32 = lane & 31;

  // ---- activation sources: direct loads, instruction j of wave w fills rows
  // 8 * (NWAVES * j + w) + lane / 8, LDS slot lane % 8
  uint32_t a_off[AJ];  // byte offset of this lane's 16-byte chunk, without the step base
#pragma unroll
  for (int j = 0; j < AJ; ++j) {
    const int row = 8 * (NWAVES * j + wave) + (lane >> 3);
    const int chunk = lds_slot(row, lane & 7);  // the slot map is an involution per row
    const int r = min(row, valid - 1);
    int src_row;
    if constexpr (GATEUP) src_row = perm[m0 + r];  // the route's token (the sort's tok array)
    else src_row = m0 + r;
    a_off[j] = 2u * (uint32_t)(src_row * Kdim + BP::coff(chunk));
  }
  // down: the output row of each of the tile's routes (-1 past its routes), loaded here and
  // put in LDS once the prologue's loads are out (so they do not wait for it); visible after
  // the prologue's barrier, read by the epilogue
  static_assert(BM <= NTHREADS, "one output row per thread");
  int orow_v = -1;
  if constexpr (!GATEUP) {
    if (tid < valid) orow_v = perm[m0 + tid];
  }
  // buffer loads into LDS: the step's column offset is a scalar operand, the lane's row
  // offset a fixed register, so no address arithmetic per load; reads beyond a_bytes
  // (never made: rows are clamped to the tile's last valid one) would return zeros
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)A_src, (short)0, a_bytes, 0x00020000);
  auto issue_a = [&](int sb, auto subc, int buf, int j0, int j1) {
    constexpr int SUB = decltype(subc)::value;
    const int sbase = 2 * (256 * sb + BP::template ksub<SUB>());
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      uint8_t* dst = a_lds + buf * A_BYTES + (8 * (NWAVES * j + wave)) * A_ROW;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, (__attribute__((address_space(3))) void*)dst, 16, (int)a_off[j],
                                               sbase, 0, 0);
    }
  };

  // ---- this lane's weight rows: row l32 of each of the wave's FI fragments
  const uint8_t* b_row[FI];
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    int64_t wr;
    if constexpr (GATEUP) {
      constexpr int FH = FI / 2;
      const int n0 = nt * (BNW / 2);
      wr = i < FH ? (int64_t)n0 + (wn * FH + i) * 32 + l32 : (int64_t)NI + n0 + (wn * FH + i - FH) * 32 + l32;
    } else {
      wr = (int64_t)nt * BNW + (wn * FI + i) * 32 + l32;
    }
    b_row[i] = wexp + wr * rb;
  }

  // LDS byte offset of this lane's activation operand in sub-step s for route fragment 0
  // (fragment j adds 32 rows; the slot depends on the row's low 4 bits only)
  int a_rd[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int q = s < 2 ? BP::off0(h) / 8 + s : BP::off1(h) / 8 + s - 2;
    a_rd[s] = (wm * FJ * 32 + l32) * A_ROW + 16 * lds_slot(l32, q);
  }

  // the accumulators start at the tile's first MFMAs, whose C operand is the constant 0
  // (the first step is peeled off the K loop): no separate zeroing of 256 AGPRs a lane
  f32x16_t acc[FI][FJ];

  // raw ring: slot (k & 1) holds the bytes of step k (loaded two steps ahead); wv[k & 1]
  // the decoded weights of step k (decoded one step ahead)
  typename BP::Raw raw[2][FI];
  typename BP::Head head[FI], head_nxt[FI];  // super-block sb's shared bytes, and sb+1's
  uint32_t wv[2][FI][16];
  const int nsb = Kdim / 256;  // super-block columns per tile, 4 steps each
  const int lsb = nsb - 1;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  // prologue: A(0), raw(0), raw(1), all that step 0 needs before its first MFMA (step j
  // issues A(j+3), then raw(j+2); step 0 also issues A(1) and A(2)). Issuing the loads of
  // three activation steps here would hold the first MFMA back by their issue time, which
  // the address unit spends at about a cycle per row touched (the Q6_K gathers most); in
  // step 0 it runs under the MFMAs (sched_barrier keeps the compiler from hoisting the
  // register loads above the direct ones)
  auto prologue = [&]() {
#pragma unroll
    for (int i = 0; i < FI; ++i) BP::load_head(b_row[i], 0, h, head[i]);
    issue_a(0, S0{}, 0, 0, AJ);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FI; ++i) BP::template load<0>(b_row[i], 0, h, grid_lds, raw[0][i]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FI; ++i) BP::template load_next<1>(b_row[i], 0, h, grid_lds, raw[1][i], raw[0][i]);
    __builtin_amdgcn_sched_barrier(0);
  };
  prologue();
  if constexpr (!GATEUP) {
    if (tid < BM) orow_lds[tid] = orow_v;
  }
  // wait for A(0) and decode step 0 (the compiler waits for its raw bytes, issued after A(0))
  static_assert(FI * BP::NLOAD2 < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(wait_vmcnt(FI * BP::NLOAD2));
  __syncthreads();  // A(0) of every wave; the codebook
#pragma unroll
  for (int i = 0; i < FI; ++i) BP::template decode<0>(head[i], raw[0][i], grid_lds, wv[0][i]);

  int abuf = 0;
  auto step = [&](int sb, auto subc, auto phasec) {
    constexpr int SUB = decltype(subc)::value;
    // 1: the tile's first step, 2: its second, 3: one of its last three (with SUB 1..3), 0: any
    // other
    constexpr int PH = decltype(phasec)::value;
    constexpr bool FIRST = PH == 1;  // C starts at 0
    // the last three steps: no loads for steps past the tile's last (L = 4 nsb - 1): step k
    // issues A(k+3) only up to k = L - 3, the raw bytes of step k+2 up to k = L - 2, the next
    // super-block's shared bytes not at all, and the last step decodes nothing
    constexpr bool TAIL = PH == 3;
    static_assert(!TAIL || SUB >= 1, "tail steps are the super-block's last three");
    constexpr bool LOAD_A = !(TAIL && SUB >= 1), LOAD_RAW = !(TAIL && SUB >= 2), DECODE = !(TAIL && SUB == 3);
    constexpr int cur = SUB & 1;
    constexpr int SUB1 = (SUB + 1) & 3, SUB2 = (SUB + 2) & 3, SUB3 = (SUB + 3) & 3;
    const int sb2 = SUB < 2 ? sb : min(sb + 1, lsb);
    const int sb3 = SUB < 1 ? sb : min(sb + 1, lsb);
    if constexpr (SUB == 1 && !TAIL) {
#pragma unroll
      for (int i = 0; i < FI; ++i) BP::load_head(b_row[i], min(sb + 1, lsb), h, head_nxt[i]);
    }
    int anext = abuf + AD - 1;
    if (anext >= AD) anext -= AD;
    const uint8_t* Ab = a_lds + abuf * A_BYTES;
    // two regions of two sub-steps; in each: half of the direct loads of A(k+3), the raw
    // bytes of one piece of step k+2 (raw[cur] held step k, decoded one step ago), the
    // reads of the next sub-steps' activation operands (double-buffered in registers), 32
    // MFMAs and one piece of the decode of step k+1, interleaved by the schedule below so
    // the matrix core never waits for a run of decode, an LDS read or a burst of gathers
    static_assert(FI == 2, "the schedule assumes 2 pieces per step");
    constexpr int NMR = 2 * FI * FJ;       // MFMAs per region
    constexpr int DSR = NMR / (2 * FJ);    // MFMAs per LDS read
    bf16x8_t af[2][FJ];
#pragma unroll
    for (int j = 0; j < FJ; ++j) af[0][j] = *(const bf16x8_t*)(Ab + j * 32 * A_ROW + a_rd[0]);
#pragma unroll
    for (int s2 = 0; s2 < 4; s2 += 2) {
      // the codebook reads (IQ3_S) of the piece this region decodes, ahead of the region's
      // activation reads: the decode then waits only for them, not for every LDS read
      const typename BP::Head& hd1 = SUB == 3 ? head_nxt[s2 / 2] : head[s2 / 2];
      typename BP::Look look;
      if constexpr (DECODE) BP::template lookup<SUB1>(hd1, raw[cur ^ 1][s2 / 2], grid_lds, look);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (FIRST) {
        // the tile's first step issues A(1), A(2) and A(3), in that order (the prologue only
        // A(0)): region 0 A(1) and the first half of A(2), region 1 the rest
        if (s2 == 0) {
          issue_a(0, S1{}, 1, 0, AJ);
          issue_a(0, S2{}, 2, 0, AJ / 2);
        } else {
          issue_a(0, S2{}, 2, AJ / 2, AJ);
          issue_a(0, S3{}, 3, 0, AJ);
        }
      } else if constexpr (LOAD_A) {
        issue_a(sb3, std::integral_constant<int, SUB3>{}, anext, (s2 / 2) * AJ / 2, (s2 / 2 + 1) * AJ / 2);
      }
      // raw[cur ^ 1] holds step k+1, the step before k+2 in the same super-block column
      if constexpr (LOAD_RAW)
        BP::template load_next<SUB2>(b_row[s2 / 2], sb2, h, grid_lds, raw[cur][s2 / 2], raw[cur ^ 1][s2 / 2]);
#pragma unroll
      for (int j = 0; j < FJ; ++j) af[1][j] = *(const bf16x8_t*)(Ab + j * 32 * A_ROW + a_rd[s2 + 1]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int s = s2 + t;
        bf16x8_t wf[FI];
#pragma unroll
        for (int i = 0; i < FI; ++i) {
          u32x4_t v = {wv[cur][i][4 * s], wv[cur][i][4 * s + 1], wv[cur][i][4 * s + 2], wv[cur][i][4 * s + 3]};
          wf[i] = __builtin_bit_cast(bf16x8_t, v);
        }
#pragma unroll
        for (int j = 0; j < FJ; ++j)
#pragma unroll
          for (int i = 0; i < FI; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                wf[i], af[t][j], FIRST && s == 0 ? f32x16_t{} : acc[i][j], 0, 0, 0);
        if (t == 0 && s2 == 0) {
#pragma unroll
          for (int j = 0; j < FJ; ++j) af[0][j] = *(const bf16x8_t*)(Ab + j * 32 * A_ROW + a_rd[2]);
        }
      }
      if constexpr (DECODE) BP::template convert<SUB1>(hd1, raw[cur ^ 1][s2 / 2], grid_lds, look, wv[cur ^ 1][s2 / 2]);
      // schedule: the direct loads first, then 32 x (1 MFMA, VPM VALU), an LDS read after
      // every other MFMA and one of the raw weight gathers after every other (each
      // gathers 32 rows' cache lines: in one burst they would hold up the MFMA issue).
      // VPM covers the type's decode (Q4_K and Q8_0 about 3.5 VALU per MFMA, Q6_K 4.1,
      // IQ3_S 4.3 once its codebook reads are out of the region): VALU left over would run
      // after the last MFMA with the matrix core idle.
      // (gate/up: the direct loads take the first of the per-MFMA VMEM slots instead of a
      // burst at the region's start: gate/up 337.5 -> 335.5 us at the sustained clock; the
      // down GEMM unchanged either way)
      if constexpr (!GATEUP) __builtin_amdgcn_sched_group_barrier(0x020, AJ / 2, 0);
#pragma unroll
      for (int m = 0; m < NMR; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, BP::VPM, 0);
        if (m % DSR == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (m % 2 == 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // A(k+1) has landed once at most the VMEM ops issued after it are outstanding: A(k+2),
    // A(k+3) and the raw bytes of steps k+1 and k+2 (NLOAD2 instructions a piece over the
    // two, the count the compiler emits; the compiler waits for those register loads itself
    // before their decode). tests/test_asm_waitcnt.py checks this count against the gfx950
    // assembly.
    // The tile's first two steps: A(1) is followed by A(2), A(3) and the raw bytes of step 2
    // (at least NLOAD2 - NLOAD instructions a piece, the smaller step of a pair); A(2) by half
    // of A(3), A(4) and step 3's raw bytes. The last three: A(L-1) by A(L) and the raw bytes
    // of steps L-1 and L; A(L) by step L's raw bytes; after step L nothing is waited for here
    // and no barrier taken (every epilogue waits for its loads itself, and the ones that reuse
    // the activation buffers synchronise the block first).
    constexpr int NYOUNG = PH == 1   ? 2 * AJ + FI * (BP::NLOAD2 - BP::NLOAD)
                           : PH == 2 ? AJ + AJ / 2 + FI * (BP::NLOAD2 - BP::NLOAD)
                           : TAIL    ? (SUB == 1 ? AJ + FI * BP::NLOAD2 : FI * (BP::NLOAD2 - BP::NLOAD))
                                     : 2 * AJ + FI * BP::NLOAD2;
    static_assert(NYOUNG > 0 && NYOUNG < 64, "vmcnt range");
    if constexpr (!(TAIL && SUB == 3)) {
      __builtin_amdgcn_s_waitcnt(wait_vmcnt(NYOUNG));
      lds_barrier();
    }
    abuf = abuf + 1 == AD ? 0 : abuf + 1;
    if constexpr (SUB == 3) {
#pragma unroll
      for (int i = 0; i < FI; ++i) head[i] = head_nxt[i];
    }
  };

  // 128-route tiles: the bf16 C tile is staged in LDS over the activation buffers (rows of
  // CW 16-byte chunks, chunk c of row r at slot c ^ (r % CW)), then written out as whole
  // rows, 16 bytes per lane (each row's segment by consecutive lanes: full cache lines per
  // instruction).
  // Accumulator layout: lane l holds route 32 j + l % 32 and weight rows
  // 8 (r / 4) + 4 (l / 32) + r % 4 of fragment i: 4 consecutive columns per (i, j, r / 4).
  constexpr int CCOLS = GATEUP ? BNW / 2 : BNW;  // output columns of a tile
  constexpr int CW = CCOLS / 8;                  // 16-byte chunks per row
  static_assert(BM * CCOLS * 2 <= AD * A_BYTES, "C tile fits the activation buffers");
  uint8_t* cs = a_lds;
  auto c_put = [&](int row, int col, uint32_t lo, uint32_t hi) {
    const int c = col >> 3;
    u32x2_t v = {lo, hi};
    *(u32x2_t*)(cs + row * (CW * 16) + 16 * (c ^ (row % CW)) + 2 * (col & 7)) = v;
  };
  constexpr int NIT = BM * CW / NTHREADS;
  static_assert(BM * CW % NTHREADS == 0, "store mapping");

  // down: the accumulators to the bf16 output rows Y[perm[m]] (streamed past the caches: Y is
  // read once, by the combine, long after)
  auto flush = [&]() {
    if constexpr (WAVE_STG && !GATEUP) {
      // per 32-route slice j: the wave's 32 x FI*32 block into its staging area (rows of
      // 128 B, chunk c of row r at slot c ^ (r % 8)), then 8 rows x 128 B per store. A
      // wave's LDS operations complete in order, so no barrier sits between the writes and
      // the reads of other lanes, nor between the reads and the next slice's writes.
      __builtin_amdgcn_s_waitcnt(0);  // the clamped prefetches of the last steps (into LDS) have landed
      uint8_t* stg = a_lds + AD * A_BYTES + OROW_BYTES + wave * STG_WAVE;
      const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, out_bytes, 0x00020000);
      const uint32_t col_b = 2u * (uint32_t)(nt * CCOLS + wn * FI * 32) + 16u * (uint32_t)(lane & 7);
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const f32x16_t& v = acc[i][j];
            const u32x2_t w = {f2bf2(v[4 * r4], v[4 * r4 + 1]), f2bf2(v[4 * r4 + 2], v[4 * r4 + 3])};
            *(u32x2_t*)(stg + l32 * 128 + 16 * ((4 * i + r4) ^ (l32 & 7)) + 8 * h) = w;
          }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const int row = 8 * it + (lane >> 3);
          const u32x4_t v = *(const u32x4_t*)(stg + row * 128 + 16 * ((lane & 7) ^ (row & 7)));
          const int orow = orow_lds[32 * j + row];
          const uint32_t off = orow >= 0 ? (uint32_t)orow * (2u * (uint32_t)NI) + col_b : 0xFFFFFFF0u;
          __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, (int)off, 0, 2);  // nt: Y is read once, much later
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    } else if constexpr (!GATEUP) {
      __builtin_amdgcn_s_waitcnt(0);  // the clamped prefetches of the last steps (into LDS)
      __syncthreads();                 // every wave is done with the activation buffers
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        const int ml = 32 * (wm * FJ + j) + l32;
#pragma unroll
        for (int i = 0; i < FI; ++i) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const f32x16_t& a = acc[i][j];
            c_put(ml, (wn * FI + i) * 32 + 8 * r4 + 4 * h, f2bf2(a[4 * r4], a[4 * r4 + 1]),
                  f2bf2(a[4 * r4 + 2], a[4 * r4 + 3]));
          }
        }
      }
      __syncthreads();
      // buffer stores with 32-bit offsets (out_bytes < 4 GiB), no branch: a row past the
      // tile's routes (orow -1) gets an offset past the buffer, and the store is dropped
      const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, out_bytes, 0x00020000);
      const uint32_t col_b = 2u * (uint32_t)(nt * CCOLS);
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int qq = tid + it * NTHREADS;
        const int ml = qq / CW, c = qq % CW;
        const int orow = orow_lds[ml];
        const u32x4_t v = *(const u32x4_t*)(cs + ml * (CW * 16) + 16 * (c ^ (ml % CW)));
        const uint32_t off = orow >= 0 ? (uint32_t)orow * (2u * (uint32_t)NI) + col_b + 16u * (uint32_t)c : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, (int)off, 0, 2);  // nt: Y is read once, much later
      }
    }
  };

  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  using P0 = std::integral_constant<int, 0>;
  using P3 = std::integral_constant<int, 3>;
  step(0, S0{}, P1{});  // nsb >= 1: the layer requires Kdim to be a multiple of 256
  step(0, S1{}, P2{});
  step(0, S2{}, P0{});
  step(0, S3{}, P0{});
  if (nsb > 1) {  // (a one-column tile keeps the clamped loads of its last steps)
    for (int sb = 1; sb < lsb; ++sb) {
      step(sb, S0{}, P0{});
      step(sb, S1{}, P0{});
      step(sb, S2{}, P0{});
      step(sb, S3{}, P0{});
    }
    step(lsb, S0{}, P0{});
    step(lsb, S1{}, P3{});
    step(lsb, S2{}, P3{});
    step(lsb, S3{}, P3{});
  }
  if constexpr (!GATEUP) {
    flush();
    return;
  }
  constexpr int FH = FI / 2;
  if constexpr (WAVE_STG) {
    // ---- gate/up epilogue, per wave: silu(gate) * up of each 32-route slice j into the
    // wave's staging area (rows of 64 B, chunk c of row r at slot c ^ sw(r): any 8 or 16
    // consecutive rows spread over the banks), then 16 rows x 64 B per store (the other
    // waves write the rest of each H row segment)
    static_assert(FH == 1, "one gate and one up fragment per wave");
    __builtin_amdgcn_s_waitcnt(0);  // the clamped prefetches of the last steps (into LDS) have landed
    uint8_t* stg = a_lds + AD * A_BYTES + OROW_BYTES + wave * STG_WAVE;
    auto sw = [](int r) { return ((r >> 1) ^ (r >> 3)) & 3; };
    const __amdgpu_buffer_rsrc_t h_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, out_bytes, 0x00020000);
    const uint32_t col_b = 2u * (uint32_t)(nt * CCOLS + wn * 32) + 16u * (uint32_t)(lane & 3);
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const f32x16_t& g = acc[0][j];
      const f32x16_t& u = acc[1][j];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const u32x2_t v = {f2bf2(silu_mul(g[4 * r4], u[4 * r4]), silu_mul(g[4 * r4 + 1], u[4 * r4 + 1])),
                           f2bf2(silu_mul(g[4 * r4 + 2], u[4 * r4 + 2]), silu_mul(g[4 * r4 + 3], u[4 * r4 + 3]))};
        *(u32x2_t*)(stg + l32 * 64 + 16 * (r4 ^ sw(l32)) + 8 * h) = v;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int row = 16 * it + (lane >> 2);
        const u32x4_t v = *(const u32x4_t*)(stg + row * 64 + 16 * ((lane & 3) ^ sw(row)));
        const int ml = 32 * j + row;
        // rows past the tile's routes get an offset past the buffer and are dropped; cached
        // (the down GEMM reads H back soon)
        const uint32_t off = ml < valid ? (uint32_t)(m0 + ml) * (2u * (uint32_t)NI) + col_b : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_buffer_store_b128(v, h_rsrc, (int)off, 0, 0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the clamped prefetches of the last steps
  __syncthreads();                 // every wave is done with the activation buffers

  // ---- gate/up epilogue: silu(gate) * up into the C tile, then whole rows of H
#pragma unroll
  for (int j = 0; j < FJ; ++j) {
    const int ml = 32 * (wm * FJ + j) + l32;
#pragma unroll
    for (int i = 0; i < FH; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x16_t& g = acc[i][j];
        const f32x16_t& u = acc[i + FH][j];
        c_put(ml, (wn * FH + i) * 32 + 8 * r4 + 4 * h,
              f2bf2(silu_mul(g[4 * r4], u[4 * r4]), silu_mul(g[4 * r4 + 1], u[4 * r4 + 1])),
              f2bf2(silu_mul(g[4 * r4 + 2], u[4 * r4 + 2]), silu_mul(g[4 * r4 + 3], u[4 * r4 + 3])));
      }
  }
  __syncthreads();
  // buffer stores with 32-bit offsets, no branch: rows past the tile's routes get an offset
  // past the buffer and are dropped; cached (the down GEMM reads H back soon)
  const __amdgpu_buffer_rsrc_t h_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, out_bytes, 0x00020000);
  const uint32_t col_b = 2u * (uint32_t)(nt * CCOLS);
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int q = tid + it * NTHREADS;
    const int ml = q / CW, c = q % CW;
    const u32x4_t v = *(const u32x4_t*)(cs + ml * (CW * 16) + 16 * (c ^ (ml % CW)));
    const uint32_t off = ml < valid ? (uint32_t)(m0 + ml) * (2u * (uint32_t)NI) + col_b + 16u * (uint32_t)c : 0xFFFFFFF0u;
    __builtin_amdgcn_raw_buffer_store_b128(v, h_rsrc, (int)off, 0, 0);
  }
}

// One block per (route tile, weight-row tile). A slot's last tile holds the slot's remaining
// routes (1..BM); at 256-route tiles (FJ = 8) one that holds at most 128 runs the 128-route
// body instead, so the padding of a slot's last tile costs at most 127 routes' MFMAs, not 255.
template <int TYPE, bool GATEUP, int FJ>
__global__ __launch_bounds__(NTHREADS, (gemm_waves_per_simd<TYPE, FJ>()))
void grouped_gemm(const uint16_t* __restrict__ A_src, uint32_t a_bytes, const int32_t* __restrict__ perm,
                  const int4* __restrict__ tile_info, int top_k, const uint8_t* __restrict__ W, int w_is_table,
                  int64_t w_expert_stride, int64_t rb, int Kdim, int NI, int NT, int64_t nblk,
                  uint16_t* __restrict__ out, uint32_t out_bytes) {
  static_assert(gemm_lds_bytes<TYPE, GATEUP, 4>() <= gemm_lds_bytes<TYPE, GATEUP, 8>(), "the 128-route body fits");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[gemm_lds_bytes<TYPE, GATEUP, FJ>()];

  // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin (pid % 8). Tile-table
  // position p = (idx / NT) * 8 + pid % 8 is on XCD pid % 8, and the table gives each XCD a
  // contiguous range of (slot-sorted) M tiles, so a slot's weights are fetched into one L2;
  // the NT N tiles of an M tile follow each other on that XCD and share the gathered rows.
  // gridDim.x is a multiple of 8 * NT; positions without a tile hold valid = 0.
  const int64_t pid = blockIdx.x;
  const int64_t idx = pid >> 3;
  const int mt = (int)((idx / NT) * 8 + (pid & 7));
  const int nt = (int)(idx % NT);
  if ((int64_t)mt * NT + nt >= nblk) return;
  const int4 ti = tile_info[mt];
  const int e = ti.x, m0 = ti.y, valid = ti.z;
  if (valid == 0) return;

  if constexpr (TYPE == GGML_IQ3_S) stage_iq3s_sel((uint32_t*)smem);
  const uint8_t* wexp = w_is_table ? (const uint8_t*)((const int64_t*)W)[e] : W + (int64_t)e * w_expert_stride;
  if constexpr (FJ == 8) {
    if (valid <= tile_m<4>()) {
      gemm_tile<TYPE, GATEUP, 4>(smem, A_src, a_bytes, perm, top_k, wexp, rb, Kdim, NI, nt, m0, valid, out, out_bytes);
      return;
    }
  }
  gemm_tile<TYPE, GATEUP, FJ>(smem, A_src, a_bytes, perm, top_k, wexp, rb, Kdim, NI, nt, m0, valid, out, out_bytes);
}

// res[t, c] = bf16( sum_{k asc, slot_ids >= 0} fp32( bf16( Y[p, c] * bf16(w[p]) ) ) ), 8 columns
// per thread. The k's go in groups of 8 (then of 2 for the rest) whose Y loads are all issued
// before the first is used: a token's rows are independent HBM reads, not round trips in a
// row. A cold route (or k past top_k) loads from offset y_bytes, past the buffer's end: the
// load returns zeros without touching memory and its weight is 0, so it adds +0.0f, which
// leaves every sum as it was (the sum starts at +0.0f and is never -0.0f).
__global__ __launch_bounds__(256) void combine_routes(const uint16_t* __restrict__ Y, uint32_t y_bytes,
                                                      const float* __restrict__ w,
                                                      const int32_t* __restrict__ slot_ids, int S, int top_k,
                                                      int64_t K, uint16_t* __restrict__ res) {
  const int64_t t = blockIdx.y;
  const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)Y, (short)0, y_bytes, 0x00020000);
  for (int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; c < K; c += (int64_t)gridDim.x * blockDim.x * 8) {
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = 0.0f;
    // routes k0 .. k0 + G - 1; with guardc true, a k past top_k reads no id or weight and is cold
    auto group = [&](int k0, auto gc, auto guardc) {
      constexpr int G = decltype(gc)::value;
      const int64_t p0 = t * top_k + k0;
      int e[G];
      float wr[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {  // loaded first, whatever e is: a whole group's loads merge
        const bool in = !decltype(guardc)::value || k0 + j < top_k;
        e[j] = in ? slot_ids[p0 + j] : -1;
        wr[j] = in ? w[p0 + j] : 0.0f;
      }
      uint32_t off[G];
      float wk[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const bool hot = e[j] >= 0 && e[j] < S;
        wk[j] = hot ? bf2f(f2bf(wr[j])) : 0.0f;
        off[j] = hot ? (uint32_t)(((p0 + j) * K + c) * 2) : y_bytes;
      }
      u32x4_t v[G];
#pragma unroll
      for (int j = 0; j < G; ++j) v[j] = __builtin_amdgcn_raw_buffer_load_b128(y_rsrc, off[j], 0, 2);  // nt: read once
      __builtin_amdgcn_sched_barrier(0);  // all G loads issued before the first is used
#pragma unroll
      for (int j = 0; j < G; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[2 * i] += bf2f(f2bf(bf2f(v[j][i] & 0xFFFF) * wk[j]));
          a[2 * i + 1] += bf2f(f2bf(bf2f(v[j][i] >> 16) * wk[j]));
        }
      }
    };
    int k0 = 0;
    for (; k0 + 8 <= top_k; k0 += 8) group(k0, std::integral_constant<int, 8>{}, std::false_type{});
    for (; k0 < top_k; k0 += 2) group(k0, std::integral_constant<int, 2>{}, std::true_type{});
    u32x4_t o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2bf2(a[2 * i], a[2 * i + 1]);
    *(u32x4_t*)(res + t * K + c) = o;
  }
}

template <int TYPE, bool GATEUP, int FJ>
void launch_gemm(dim3 grid, hipStream_t stream, const uint16_t* A_src, uint32_t a_bytes, const int32_t* perm,
                 const int4* tile_info, int top_k, const void* W, int w_is_table, int64_t w_expert_stride, int64_t rb,
                 int Kdim, int NI, int NT, int64_t nblk, uint16_t* out, uint32_t out_bytes) {
  grouped_gemm<TYPE, GATEUP, FJ><<<grid, NTHREADS, 0, stream>>>(A_src, a_bytes, perm, tile_info, top_k,
                                                               (const uint8_t*)W, w_is_table, w_expert_stride, rb,
                                                               Kdim, NI, NT, nblk, out, out_bytes);
}

template <bool GATEUP, int TYPE>
void launch_fj(int fj, dim3 grid, hipStream_t stream, const uint16_t* A_src, uint32_t a_bytes,
               const int32_t* perm, const int4* tile_info, int top_k, const void* W, int w_is_table,
               int64_t w_expert_stride, int64_t rb, int Kdim, int NI, int NT, int64_t nblk, uint16_t* out,
               uint32_t out_bytes) {
  if (fj == 8)
    launch_gemm<TYPE, GATEUP, 8>(grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table,
                                 w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes);
  else
    launch_gemm<TYPE, GATEUP, 4>(grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table,
                                 w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes);
}

template <bool GATEUP>
int dispatch_gemm(int type, int fj, dim3 grid, hipStream_t stream, const uint16_t* A_src, uint32_t a_bytes,
                  const int32_t* perm, const int4* tile_info, int top_k, const void* W, int w_is_table,
                  int64_t w_expert_stride, int64_t rb, int Kdim, int NI, int NT, int64_t nblk, uint16_t* out,
                  uint32_t out_bytes) {
  switch (type) {
    case GGML_Q8_0: launch_fj<GATEUP, GGML_Q8_0>(fj, grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes); break;
    case GGML_Q4_K: launch_fj<GATEUP, GGML_Q4_K>(fj, grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes); break;
    case GGML_Q6_K: launch_fj<GATEUP, GGML_Q6_K>(fj, grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes); break;
    case GGML_IQ3_S: launch_fj<GATEUP, GGML_IQ3_S>(fj, grid, stream, A_src, a_bytes, perm, tile_info, top_k, W, w_is_table, w_expert_stride, rb, Kdim, NI, NT, nblk, out, out_bytes); break;
    default: set_error("grouped GEMM: ggml type %d has no kernel", type); return KTMI_ETYPE;
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

// Route-tile height (FJ fragments of 32 routes): 256 routes when the gate/up GEMM then has
// about two blocks per CU of the 256, counting every route as hot (R / 256 + S tiles of NT
// gate/up column tiles), else 128: small chunks trade MFMA work per decoded weight for
// blocks that fill the chip (Q8_0 at 512 tokens: 0.106 -> 0.087 ms; Q4_K/Q6_K at 2048
// tokens: 0.204 -> 0.170 ms). 64-route tiles measured slower than either.
int grouped_fj(int64_t routes, int64_t n_slots, int64_t inter) {
  const int64_t nt13 = inter / (BNW / 2);
  return (routes / 256 + n_slots) * nt13 >= 2 * 256 ? 8 : 4;
}

GroupedPlan grouped_plan(int64_t tokens, int64_t top_k, int64_t n_slots, int64_t hidden, int64_t inter) {
  GroupedPlan P{};
  P.routes = tokens * top_k;
  P.n_slots = n_slots;
  P.fj = grouped_fj(P.routes, n_slots, inter);
  P.bm = 32 * WM * P.fj;
  const int64_t nch = (P.routes + CHW - 1) / CHW;
  P.max_tiles = ((P.routes + P.bm - 1) / P.bm + n_slots + 7) / 8 * 8;  // tile-table positions, 8 per XCD round
  int64_t o = 0;
  P.off_counts = o; o = align256(o + ((nch > 0 ? nch : 1) * n_slots + n_slots) * 4);
  P.off_seg = o; o = align256(o + (n_slots + 1) * 4);
  P.off_tseg = o; o = align256(o + (n_slots + 1) * 4);
  P.off_tinfo = o; o = align256(o + P.max_tiles * 16);
  P.off_perm = o; o = align256(o + P.routes * 4);
  P.off_tok = o; o = align256(o + P.routes * 4);
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
  // x, H and Y are addressed by buffer instructions with 32-bit offsets, 0xFFFFFFF0 marking a
  // dropped store (the caller splits longer layers into passes that fit)
  KTMI_REQUIRE(tokens * K * 2 <= 0xFFFF0000ll && R * N * 2 <= 0xFFFF0000ll && R * K * 2 <= 0xFFFF0000ll, KTMI_EINVAL,
               "grouped layer: a pass of %lld tokens exceeds the 32-bit buffer range", (long long)tokens);
  if (tokens == 0) return KTMI_OK;
  int32_t* hist = (int32_t*)(ws + P.off_counts);
  int32_t* seg = (int32_t*)(ws + P.off_seg);
  int32_t* tseg = (int32_t*)(ws + P.off_tseg);
  int32_t* perm = (int32_t*)(ws + P.off_perm);
  int32_t* tok = (int32_t*)(ws + P.off_tok);
  int4* tile_info = (int4*)(ws + P.off_tinfo);
  uint16_t* H = (uint16_t*)(ws + P.off_h);
  uint16_t* Y = (uint16_t*)(ws + P.off_y);
  const int64_t nch = (R + CHW - 1) / CHW;
  int32_t* tot = hist + nch * S;
  const unsigned sblocks = (unsigned)((nch + 3) / 4);
  record_stage(0, stream);
  if (sort_small_fits(R, S)) {
    sort_small<<<1, SMALL_THREADS, (unsigned)((nch + SMALL_WAVES) * S * 4), stream>>>(
        slot_ids, (int)R, S, (int)nch, seg, tseg, tile_info, P.max_tiles, (int)P.bm, (int)top_k, perm, tok);
  } else {
    sort_count<<<sblocks, SORT_THREADS, 0, stream>>>(slot_ids, R, S, hist, nch);
    sort_scan_chunks<<<S, SORT_THREADS, 0, stream>>>(hist, nch, tot);
    sort_scatter<<<sblocks, SORT_THREADS, 0, stream>>>(slot_ids, R, S, hist, nch, tot, seg, tseg, tile_info,
                                                       P.max_tiles, (int)P.bm, (int)top_k, perm, tok);
  }
  KTMI_HIP_TRY(hipGetLastError());
  record_stage(1, stream);
  const int64_t rb13 = row_bytes(K, L->type13), rb2 = row_bytes(N, L->type2);
  const int64_t st13 = 2 * N * rb13, st2 = K * rb2;
  const int NT1 = (int)(N / (BNW / 2));
  const int64_t nblk1 = P.max_tiles * NT1;
  dim3 g1((unsigned)((nblk1 + 8 * NT1 - 1) / (8 * NT1) * (8 * NT1)));
  int rc = dispatch_gemm<true>(L->type13, P.fj, g1, stream, x, (uint32_t)(tokens * K * 2), tok, tile_info,
                               (int)top_k, L->w13, L->w_is_table, st13, rb13, (int)K, (int)N, NT1, nblk1, H,
                               (uint32_t)(R * N * 2));
  if (rc) return rc;
  record_stage(2, stream);  // no mid stage on this path: SiLU*mul is in the gate/up epilogue
  record_stage(3, stream);
  const int NT2 = (int)(K / BNW);
  const int64_t nblk2 = P.max_tiles * NT2;
  dim3 g2((unsigned)((nblk2 + 8 * NT2 - 1) / (8 * NT2) * (8 * NT2)));
  rc = dispatch_gemm<false>(L->type2, P.fj, g2, stream, H, (uint32_t)(R * N * 2), perm, tile_info, (int)top_k,
                            L->w2, L->w_is_table, st2, rb2, (int)N, (int)K, NT2, nblk2, Y, (uint32_t)(R * K * 2));
  if (rc) return rc;
  record_stage(4, stream);
  for (int64_t t0 = 0; t0 < tokens; t0 += 65535) {
    const int64_t nt = tokens - t0 < 65535 ? tokens - t0 : 65535;
    dim3 gc((unsigned)((K / 8 + 255) / 256), (unsigned)nt);
    combine_routes<<<gc, 256, 0, stream>>>(Y + t0 * top_k * K, (uint32_t)(nt * top_k * K * 2), topk_w + t0 * top_k,
                                           slot_ids + t0 * top_k, S, (int)top_k, K, y + t0 * K);
  }
  record_stage(5, stream);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

}  // namespace ktmi
