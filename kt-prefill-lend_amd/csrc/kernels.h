// Host-side launchers shared between the kernel files and the C entry points.
#pragma once
#include "ktmi_common.h"

namespace ktmi {

int launch_dequant(const uint8_t* raw, int64_t raw_stride, int type, int64_t n, int64_t rows, int64_t cols,
                   uint16_t* out, int64_t out_stride, hipStream_t stream);
int launch_route(const int32_t* ids, int64_t n, const int32_t* log2slot, const int32_t* log2cpu, float* counts,
                 int32_t* slot_ids, int32_t* cpu_ids, hipStream_t stream);
int launch_quantize_q8_1(const void* x, int dtype, int64_t cols, int64_t tokens, uint8_t* out, hipStream_t stream);
int launch_silu_and_mul(const void* h, int dtype, int64_t R, int64_t N, void* out, hipStream_t stream);
int launch_combine(const void* out, int dtype, const float* w, int64_t T, int64_t top_k, int64_t K, void* res,
                   hipStream_t stream);

// GEMV over raw GGUF rows against q8_1 activations (the decode-window kernel).
// xq: q8_1 rows of the tokens, xq_stride bytes apart. W: slot tensor (w_is_table = 0,
// experts w_expert_stride bytes apart) or int64 table of per-slot addresses. Expert ids
// outside [0, n_experts) give zero rows like ids < 0.
int launch_moe_gemv(const uint8_t* xq, int64_t xq_stride, const void* W, int w_is_table, int64_t w_expert_stride,
                    const int32_t* ids, int64_t top_k, int64_t n_routes, int type, int64_t rows, int64_t cols,
                    void* Y, int y_dtype, int per_route, int n_experts, hipStream_t stream);

// Optional stage timing: when set (ktmi_set_stage_events), the layer records events[i]
// on its stream at each stage boundary (KTMI_STAGE_EVENTS of them).
void record_stage(int i, hipStream_t stream);

// Fused decode-sized layer (decode_layer.hip): two launches, for up to DEC_MAX_ROUTES
// routes, DEC_MAX_SLOTS slots and hidden sizes whose q8_1 rows fit DEC_MAX_XQ_LDS; the
// stage-by-stage GEMV sequence covers the rest.
constexpr int DEC_MAX_ROUTES = 256;
constexpr int DEC_MAX_SLOTS = 512;
constexpr int DEC_MAX_XQ_LDS = 48 * 1024;
bool decode_layer_fits(const ktmi_layer* L, int64_t tokens, int64_t top_k);
int64_t decode_layer_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k);
int launch_decode_layer(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                        int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream);

// Decode-sized layer on the matrix cores (decode_mfma.hip): two launches for up to
// DM_MAX_ROUTES routes of at most DM_MAX_TOKENS tokens; a down wave stages 16 rows of a slot
// in an LDS region of DM_DOWN_WAVE_LDS bytes.
constexpr int DM_MAX_ROUTES = 256;
constexpr int DM_MAX_TOKENS = 64;
constexpr int DM_DOWN_WAVE_LDS = 10 * 1024;
constexpr int DM_GU_LDS = 40 * 1024;  // gate/up: the block's 16 gate and 16 up rows
bool decode_mfma_fits(const ktmi_layer* L, int64_t tokens, int64_t top_k);
int64_t decode_mfma_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k);
int launch_decode_mfma(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                       int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, hipStream_t stream);

// Grouped prefill path (moe_gemm.hip).
struct GroupedPlan {
  int64_t routes;      // tokens * top_k
  int64_t n_slots;
  int64_t max_tiles;   // upper bound of M tiles over all slots
  int fj;              // route fragments of 32 per wave (the kernel's FJ)
  int64_t bm;          // routes per M tile (32 fj)
  // workspace carve-up (byte offsets)
  int64_t off_counts, off_seg, off_tseg, off_tinfo, off_perm, off_tok, off_h, off_y, total;
};
GroupedPlan grouped_plan(int64_t tokens, int64_t top_k, int64_t n_slots, int64_t hidden, int64_t inter);
int launch_grouped_layer(const ktmi_layer* L, const uint16_t* x, const float* topk_w, const int32_t* slot_ids,
                         int64_t tokens, int64_t top_k, uint16_t* y, uint8_t* ws, const GroupedPlan& P,
                         hipStream_t stream);

}  // namespace ktmi
