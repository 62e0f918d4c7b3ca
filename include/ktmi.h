/* ktmi: MI355X (gfx950) hot-expert MoE for GGUF experts -- the C ABI.
 *
 * Every entry point takes plain pointers (device pointers unless stated otherwise),
 * sizes and a HIP stream passed as `void*` (NULL = the default stream), returns an int
 * status (KTMI_OK or a negative KTMI_E* code) and never synchronises the stream. After a
 * failure ktmi_last_error() describes it (thread-local). Nothing here allocates device
 * memory except where stated (the streamer's device slots): scratch comes in through a
 * caller-provided workspace whose size the matching *_workspace() call returns.
 *
 * Citations name the reference interface each entry replaces; paths are relative to the
 * reference repository, P:<n> is line n of
 * trees/flash-next-gguf/sglang-v0.5.19-flash-next-gguf.patch.
 */
#ifndef KTMI_H
#define KTMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KTMI_OK 0
#define KTMI_EINVAL (-1) /* bad shape, pointer or argument */
#define KTMI_ETYPE (-2)  /* ggml type without a kernel here */
#define KTMI_EHIP (-3)   /* a HIP runtime call failed */
#define KTMI_ESPACE (-4) /* workspace smaller than required */

/* activation / output element types */
#define KTMI_F32 0
#define KTMI_F16 1
#define KTMI_BF16 2

/* ggml type ids with kernels: Q8_0 = 8, Q4_K = 12, Q6_K = 14, IQ3_S = 21 */

/* layer modes for ktmi_moe_layer */
#define KTMI_MODE_AUTO 0
#define KTMI_MODE_GEMV 1    /* decode windows: int8 dot-product GEMV over raw blocks and q8_1
                               activations (the reference kernels' numerics) */
#define KTMI_MODE_GROUPED 2 /* prefill chunks: routes sorted by slot, weights dequantised into
                               bf16 MFMA operands */
#define KTMI_MODE_DECODE 3  /* decode windows (at most 256 routes of 64 tokens): weights
                               dequantised into bf16 MFMA operands, a slot's routes as the
                               matrix columns, fp32 sums (within the layer tolerance of the
                               GEMV mode, not bit-equal to it) */

/* Thread-local text of the last failure ("" if none). */
const char* ktmi_last_error(void);

/* Library version (major*10000 + minor*100 + patch). */
int ktmi_version(void);

/* 1 if `ggml_type` has kernels here, else 0. Replaces the MMVQ_TYPES / DENSE_TYPES
 * membership checks of hot/kt_gguf_hot.py:81,187-190 and hot/kt_gguf_moe_multi.py:49. */
int ktmi_type_supported(int ggml_type);

/* Bytes of one row of `cols` values of `ggml_type`; 0 if cols is not a multiple of the
 * block size or the type is unknown. hot/kt_gguf_hot.py:88-91 (_row_bytes). */
int64_t ktmi_row_bytes(int64_t cols, int ggml_type);

/* ---- activation quantisation (q8_1) ---------------------------------------------
 * Bytes of one q8_1 row: cols padded to a multiple of 512, 36 bytes per 32 values.
 * kt_gguf_moe_multi.cu:664-668 (quant_X allocation). */
int64_t ktmi_q8_1_row_bytes(int64_t cols);
/* x [tokens, cols] (x_dtype) -> q8_1 blocks [tokens, ktmi_q8_1_row_bytes(cols)]:
 * d = amax/127, q = roundf(x/d), ds = (half d, half sum). hot/kt_gguf_moe_multi/
 * kt_gguf_moe_multi.cu:600-650 (quantize_q8_1, quantize_row_q8_1_cuda). */
int ktmi_quantize_q8_1(const void* x, int x_dtype, int64_t cols, int64_t tokens, void* out, void* stream);

/* ---- the GGUF MoE GEMV (decode windows) -------------------------------------------
 * Y[p, r] = sum over the blocks of row r of expert ids[p] of the int8 dot products
 * against q8_1(X[p / top_k]), for every route p < tokens*top_k; ids[p] < 0 gives a zero
 * row. per_route = 0: the first route of each expert computes every route of that
 * expert (one read of its weights per call); per_route = 1: each route alone. The sums
 * are the same in both. W: w_is_table = 0 -> slot tensor uint8 [E, rows, row_bytes(cols)];
 * w_is_table = 1 -> int64 [E] device table of per-slot row-0 addresses.
 * Y [tokens*top_k, rows] in x_dtype. Workspace: ktmi_moe_a8_vec_workspace(cols, tokens).
 * Replaces torch::Tensor kt_moe_a8_vec_multi(X, W, topk_ids, top_k, type, row, tokens)
 * (hot/kt_gguf_moe_multi/kt_gguf_moe_multi.cu:653-935) in both its window build and its
 * KT_PER_ROUTE / KT_PTR_TABLE builds (hot/kt_gguf_moe_multi.py:55-87). */
int64_t ktmi_moe_a8_vec_workspace(int64_t cols, int64_t tokens);
int ktmi_moe_a8_vec(const void* X, int x_dtype, int64_t cols, const void* W, int w_is_table,
                    const int32_t* ids, int64_t top_k, int ggml_type, int64_t rows, int64_t tokens,
                    int per_route, void* Y, void* workspace, int64_t ws_bytes, void* stream);

/* ---- dequantisation ---------------------------------------------------------------
 * raw: n experts, raw_stride bytes apart, each rows*row_bytes(cols) bytes of blocks;
 * out: bf16 [n, rows, cols], out_stride elements between experts, rows contiguous.
 * Replaces dequant_experts(raw, raw_stride, type_id, n, rows, cols, out)
 * (P:11471-11498; _iq3_s_kernel P:11397-11420) and extends it to Q8_0, Q4_K, Q6_K. */
int ktmi_dequant_experts(const void* raw, int64_t raw_stride, int ggml_type, int64_t n, int64_t rows,
                         int64_t cols, void* out_bf16, int64_t out_stride, void* stream);

/* ---- hot-expert registry lookups -------------------------------------------------
 * For one layer: slot_ids[i] = log2slot[ids[i]], cpu_ids[i] = log2cpu[ids[i]],
 * counts[ids[i]] += 1 (fp32, exact for counts < 2^24), i < n; ids must lie in [0, E).
 * Any n (the reference's fused kernel takes <= 64 routes, then falls back to torch).
 * Replaces HotCache.route (hot/kt_hot_cache.py:121-143) and _route_kernel (:62-75). */
int ktmi_hot_route(const int32_t* ids, int64_t n, const int32_t* log2slot, const int32_t* log2cpu,
                   float* counts, int32_t* slot_ids, int32_t* cpu_ids, void* stream);

/* ---- epilogues ---------------------------------------------------------------------
 * h [R, 2N] (rows [gate | up]) -> out [R, N] = silu(gate) * up, fp32 maths, one rounding.
 * Replaces sgl_kernel.silu_and_mul (call at hot/kt_gguf_hot.py:260). */
int ktmi_silu_and_mul(const void* h, int dtype, int64_t R, int64_t N, void* out, void* stream);

/* res[t] = round( sum_{k ascending} fp32( round( out[t,k] * round(w[t,k]) ) ) ), where
 * round() is to `dtype` (bf16/f16) and the sum is fp32. out [T, top_k, K], w fp32 [T, top_k].
 * Replaces _combine (hot/kt_gguf_hot.py:43-71) and out.mul_(w) + moe_sum (:300-304). */
int ktmi_combine(const void* out, int dtype, const float* w, int64_t T, int64_t top_k, int64_t K,
                 void* res, void* stream);

/* ---- one hot-expert MoE layer -----------------------------------------------------
 * The GPU half of a layer: routes (t, k) with slot_ids[t*top_k+k] >= 0 run the expert in
 * that slot; y[t] = combine over k of (silu(x_t Wg^T) * (x_t Wu^T)) Wd^T * w[t,k], cold
 * routes (< 0, the CPU's) contribute nothing. Deterministic (no atomics on outputs).
 * w13: slot tensor uint8 [n_slots, 2*inter, row_bytes(hidden, type13)], rows [gate; up];
 * w2: uint8 [n_slots, hidden, row_bytes(inter, type2)]; with w_is_table = 1 both are int64
 * device tables of per-slot addresses. x, y bf16 [tokens, hidden]; topk_w fp32.
 * Replaces KTGGUFHotExpertsMethod.apply (hot/kt_gguf_hot.py:240-304) and the streamer's
 * per-group dequant + cutlass_fused_moe body (P:40789-40819). */
typedef struct ktmi_layer {
  int64_t hidden;  /* K */
  int64_t inter;   /* N, the expert intermediate size (this rank's part) */
  int64_t n_slots; /* E_gpu, hot-expert slots */
  int32_t type13;  /* ggml type of gate and up */
  int32_t type2;   /* ggml type of down */
  const void* w13;
  const void* w2;
  int32_t w_is_table;
  int32_t reserved;
} ktmi_layer;

int64_t ktmi_moe_layer_workspace(const ktmi_layer* layer, int64_t tokens, int64_t top_k, int mode);
int ktmi_moe_layer(const ktmi_layer* layer, const void* x, const float* topk_w, const int32_t* slot_ids,
                   int64_t tokens, int64_t top_k, void* y, void* workspace, int64_t ws_bytes, int mode,
                   void* stream);
/* The mode KTMI_MODE_AUTO picks for this many routes: GROUPED above 256 routes, DECODE from
 * 64 routes where it applies, else GEMV. */
int ktmi_moe_layer_mode(const ktmi_layer* layer, int64_t tokens, int64_t top_k);
/* Tokens per pass of KTMI_MODE_GROUPED: a longer call runs as consecutive passes over token
 * slices of this size (each token's output depends only on its own routes), and the
 * workspace covers one pass. The grouped kernels address x [T, hidden], H [T top_k, inter]
 * and Y [T top_k, hidden] (bf16) with 32-bit offsets, so a pass is the largest multiple of
 * 256 tokens with 2 top_k max(hidden, inter) T < 4 GiB - 64 KiB: 37376 tokens at hidden 7168
 * and top-8, 130816 at hidden 2048 and top-8. No counterpart in the reference, whose torch
 * path has no such limit. */
int64_t ktmi_moe_layer_pass_tokens(const ktmi_layer* layer, int64_t top_k);

/* ktmi_moe_layer without a workspace argument. No counterpart in the reference: this is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The workspace is a library-owned device array of
 * KTMI_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call whose workspace
 * (ktmi_moe_layer_workspace) is larger fails with KTMI_ESPACE. It allocates nothing. Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU (two streams or
 * two threads without ordering between them) race. */
#define KTMI_NOALLOC_SCRATCH_BYTES (64ll << 20)
int ktmi_moe_layer_noalloc(const ktmi_layer* layer, const void* x, const float* topk_w, const int32_t* slot_ids,
                           int64_t tokens, int64_t top_k, void* y, int mode, void* stream);

/* Stage timing for benchmarks (no counterpart in the reference, whose per-layer timers are
 * host-side, P:40981-40985). events: KTMI_STAGE_EVENTS hipEvent_t handles that the next
 * ktmi_moe_layer calls on this thread record on their stream at the stage boundaries:
 * [0] start, [1] gate/up start (after route sort or x quantisation), [2] gate/up end,
 * [3] down start (after SiLU*mul + q8_1 on the GEMV path), [4] down end, [5] combine end.
 * A NULL entry is not recorded. events = NULL or n = 0 turns it off. */
#define KTMI_STAGE_EVENTS 6
int ktmi_set_stage_events(void* const* events, int n);

/* ---- host-side GGUF quantisers (CPU) --------------------------------------------
 * x fp32 [rows, cols] (host) -> blocks [rows, row_bytes(cols, type)] (host), using
 * `threads` CPU threads (<= 0: all). Q8_0 d = amax/127; Q4_K/Q6_K per-sub-block range
 * scales; IQ3_S nearest codebook point per 4-value group. Used to build expert weights;
 * the GGUF files the reference loads are produced by llama.cpp's quantisers. */
int ktmi_quantize_rows_host(const float* x, int64_t rows, int64_t cols, int ggml_type, void* out, int threads);

/* ---- layer-weight streamer (P:40543-40550 _Slot, P:40773-40787 _stage, P:40928-40992 run).
 * Experts' raw GGUF bytes move from pinned host banks into double-buffered device slots on
 * a copy stream of its own while the compute stream runs the grouped layer on the other
 * slot. A slot holds up to max_group experts as w13 [n, 2N, row bytes] (gate rows, then up
 * rows) and w2 [n, K, row bytes]: the layout ktmi_layer reads (hot/kt_gguf_hot.py:17-21). */
#define KTMI_STREAM_MAX_SLOTS 4
typedef struct ktmi_streamer ktmi_streamer;

/* One layer's pinned host copy of n_experts experts, one array per projection with each
 * expert's bytes contiguous: the reference's _bank (P:40700-40752, [E, part bytes]). */
typedef struct ktmi_bank {
  const void* gate; /* host [n_experts, part_gate] */
  const void* up;   /* host [n_experts, part_up]; part_up == part_gate */
  const void* down; /* host [n_experts, part_down] */
  int64_t part_gate, part_up, part_down;
  int64_t n_experts;
} ktmi_bank;

/* Allocates n_slots (2..KTMI_STREAM_MAX_SLOTS) device slots of max_group experts
 * (part13 = gate + up bytes and part2 = down bytes per expert) and the copy stream, on the
 * current device. Replaces preallocate() / _Slot (P:40607-40636, 40543-40550). NULL on
 * failure (ktmi_last_error). */
ktmi_streamer* ktmi_streamer_create(int64_t max_group, int64_t part13, int64_t part2, int n_slots);
int ktmi_streamer_destroy(ktmi_streamer* s);
/* device pointers of slot `slot`'s w13 and w2 */
int ktmi_streamer_slot(ktmi_streamer* s, int slot, void** w13, void** w2);
/* Copies experts [first, first+n) of `bank` into `slot` on the copy stream, after the
 * compute stream's last release of the slot; the slot's loaded event follows the copies.
 * Replaces _stage (P:40773-40787). */
int ktmi_streamer_stage(ktmi_streamer* s, int slot, const ktmi_bank* bank, int64_t first, int64_t n);
/* `stream` waits until the slot's last staging has landed (cur.wait_event(dma_done), P:40976). */
int ktmi_streamer_acquire(ktmi_streamer* s, int slot, void* stream);
/* marks the slot free once `stream` reaches this point (compute_done.record, P:40978) */
int ktmi_streamer_release(ktmi_streamer* s, int slot, void* stream);
/* host wait for every copy staged so far */
int ktmi_streamer_sync(ktmi_streamer* s);
/* the copy stream (hipStream_t), e.g. to time the copies with events on it */
void* ktmi_streamer_copy_stream(ktmi_streamer* s);
/* out[i] = ids[i] - base if base <= ids[i] < base + count, else -1: a group's local slot
 * ids (the reference's `local`, P:40798). */
int ktmi_remap_ids(const int32_t* ids, int64_t n, int32_t base, int32_t count, int32_t* out, void* stream);
/* acc[i] = bf16(acc[i] + x[i]) for bf16 arrays (acc.add_(out), P:40819); 16-byte aligned */
int ktmi_add_bf16(void* acc, const void* x, int64_t n, void* stream);
/* pinned host memory for banks (hipHostMalloc; the reference pins through kt_pinned,
 * P:39462-39586). NULL on failure. */
void* ktmi_host_alloc(int64_t bytes);
int ktmi_host_free(void* p);

/* ---- CPU cold experts and the GPU <-> CPU handoff.
 * The engine computes a layer's routes to CPU experts on the host cores with the numerics of
 * kt-kernel's LLAMAFILE MoE forward_many (K:2571-2800): x quantised to Q8_K (Q8_0 for Q8_0
 * weights), int8 block dot products, silu(gate)*up in fp32 re-quantised for down, fp32
 * weighted sum in route order, one bf16 rounding. Its weights are a bank of every expert
 * (ktmi_bank, host memory that outlives the engine); expert ids index the bank, other ids
 * (-1 for the GPU's residents) add nothing. Types: 8, 12, 14, 21. */
typedef struct ktmi_cpu_moe ktmi_cpu_moe;
/* threads <= 0: the CPUs of the process affinity mask, minus one. max_tokens x max_top_k sizes the pinned staging
 * of submit (0 for a forward-only engine). Replaces kt-kernel's MOE construction and
 * KExpertsCPUBuffer (the wrapper's CPU side). NULL on failure. */
ktmi_cpu_moe* ktmi_cpu_moe_create(int64_t hidden, int64_t inter, int type13, int type2, const ktmi_bank* bank,
                                  int threads, int64_t max_tokens, int64_t max_top_k);
int ktmi_cpu_moe_destroy(ktmi_cpu_moe* h);
/* Host arrays: x_bf16 [tokens, hidden], expert_ids int32 [tokens, top_k], weights fp32,
 * out_bf16 [tokens, hidden]; synchronous (forward_many). */
int ktmi_cpu_moe_forward(ktmi_cpu_moe* h, int64_t tokens, int64_t top_k, const int32_t* expert_ids,
                         const float* weights, const void* x_bf16, void* out_bf16);
/* Device arrays on `stream`: staged to pinned host memory after the stream's prior work,
 * then computed by the engine's worker thread while the stream continues. Replaces
 * BaseMoEWrapper.submit_forward and kt_uva_handoff.submit (P:10590-10602, P:41240-41270). */
int ktmi_cpu_moe_submit(ktmi_cpu_moe* h, const void* x_bf16, const int32_t* expert_ids, const float* weights,
                        int64_t tokens, int64_t top_k, void* stream);
/* Waits (host) for the submitted layer, then out_bf16 = bf16(out_bf16 + cpu output) on
 * `stream` (16-byte aligned). Replaces sync_forward + `output + cpu_output` and
 * kt_uva_handoff.sync_add (P:10598-10602, P:41285-41301). */
int ktmi_cpu_moe_sync_add(ktmi_cpu_moe* h, void* out_bf16, void* stream);
int ktmi_cpu_moe_threads(const ktmi_cpu_moe* h);
/* The bound (microseconds, default 10 s) on how long the add that sync_add enqueues ahead of
 * a decode window's CPU side waits for it. An add that waits longer writes NaN into the
 * layer's rows, exits, and sync_add returns KTMI_EHIP. No counterpart in the reference,
 * whose add waits without a bound (sync_with_cuda_stream, P:41294). Not while a submit is
 * outstanding. */
int ktmi_cpu_moe_set_add_wait(ktmi_cpu_moe* h, int64_t microseconds);
/* "avx512-vnni" or "scalar": the engine's int8 dot-product kernels (VNNI when the host has
 * it, unless KTMI_CPU_ISA=scalar was set at creation) */
const char* ktmi_cpu_moe_isa(const ktmi_cpu_moe* h);

#ifdef __cplusplus
}
#endif

#endif /* KTMI_H */
