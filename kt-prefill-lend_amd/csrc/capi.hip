// extern "C" entry points of libktmi.so: argument checks, workspace carve-up, dispatch.
#include <mutex>

#include <stdarg.h>
#include <stdio.h>

#include "kernels.h"

namespace ktmi {

static thread_local char g_err[512] = "";

void clear_error() { g_err[0] = 0; }

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

static bool type_ok(int t) { return t == GGML_Q8_0 || t == GGML_Q4_K || t == GGML_Q6_K || t == GGML_IQ3_S; }
static bool dtype_ok(int d) { return d == KTMI_F32 || d == KTMI_F16 || d == KTMI_BF16; }
static bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

static thread_local hipEvent_t g_stage_events[KTMI_STAGE_EVENTS];
static thread_local int g_stage_on = 0;

void record_stage(int i, hipStream_t stream) {
  if (g_stage_on && i >= 0 && i < KTMI_STAGE_EVENTS && g_stage_events[i]) (void)hipEventRecord(g_stage_events[i], stream);
}

// routes per call above which KTMI_MODE_AUTO takes the grouped MFMA path
static const int64_t kGemvMaxRoutes = 256;

}  // namespace ktmi

using namespace ktmi;

extern "C" {

const char* ktmi_last_error(void) { return g_err; }

int ktmi_version(void) { return 100; }

int ktmi_set_stage_events(void* const* events, int n) {
  g_err[0] = 0;
  if (n == 0 || events == nullptr) {
    g_stage_on = 0;
    return KTMI_OK;
  }
  KTMI_REQUIRE(n == KTMI_STAGE_EVENTS, KTMI_EINVAL, "set_stage_events: %d events (need %d)", n, KTMI_STAGE_EVENTS);
  for (int i = 0; i < n; ++i) g_stage_events[i] = (hipEvent_t)events[i];
  g_stage_on = 1;
  return KTMI_OK;
}

int ktmi_type_supported(int ggml_type) { return type_ok(ggml_type) ? 1 : 0; }

int64_t ktmi_row_bytes(int64_t cols, int ggml_type) {
  if (!type_ok(ggml_type) || cols <= 0 || cols % blck_size(ggml_type)) return 0;
  return row_bytes(cols, ggml_type);
}

int64_t ktmi_q8_1_row_bytes(int64_t cols) { return cols > 0 ? q8_1_row_bytes(cols) : 0; }

int ktmi_quantize_q8_1(const void* x, int x_dtype, int64_t cols, int64_t tokens, void* out, void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(dtype_ok(x_dtype), KTMI_EINVAL, "quantize_q8_1: dtype %d", x_dtype);
  KTMI_REQUIRE(cols > 0 && tokens >= 0, KTMI_EINVAL, "quantize_q8_1: cols %lld tokens %lld", (long long)cols,
               (long long)tokens);
  KTMI_REQUIRE(tokens == 0 || (x && out && aligned(out, 4)), KTMI_EINVAL, "quantize_q8_1: null or misaligned pointer");
  return launch_quantize_q8_1(x, x_dtype, cols, tokens, (uint8_t*)out, (hipStream_t)stream);
}

int64_t ktmi_moe_a8_vec_workspace(int64_t cols, int64_t tokens) {
  if (cols <= 0 || tokens < 0) return 0;
  return q8_1_row_bytes(cols) * tokens;
}

int ktmi_moe_a8_vec(const void* X, int x_dtype, int64_t cols, const void* W, int w_is_table, const int32_t* ids,
                    int64_t top_k, int ggml_type, int64_t rows, int64_t tokens, int per_route, void* Y,
                    void* workspace, int64_t ws_bytes, void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(type_ok(ggml_type), KTMI_ETYPE, "moe_a8_vec: ggml type %d has no kernel", ggml_type);
  KTMI_REQUIRE(dtype_ok(x_dtype), KTMI_EINVAL, "moe_a8_vec: dtype %d", x_dtype);
  KTMI_REQUIRE(cols > 0 && cols % blck_size(ggml_type) == 0, KTMI_EINVAL,
               "moe_a8_vec: cols %lld not a multiple of the block size %lld", (long long)cols,
               (long long)blck_size(ggml_type));
  KTMI_REQUIRE(rows > 0 && top_k > 0 && tokens >= 0, KTMI_EINVAL, "moe_a8_vec: rows %lld top_k %lld tokens %lld",
               (long long)rows, (long long)top_k, (long long)tokens);
  KTMI_REQUIRE(tokens * top_k <= 65535, KTMI_EINVAL, "moe_a8_vec: %lld routes (at most 65535 per call)",
               (long long)(tokens * top_k));
  if (tokens == 0) return KTMI_OK;
  const int64_t need = ktmi_moe_a8_vec_workspace(cols, tokens);
  KTMI_REQUIRE(workspace && ws_bytes >= need, KTMI_ESPACE, "moe_a8_vec: workspace %lld < %lld bytes",
               (long long)ws_bytes, (long long)need);
  KTMI_REQUIRE(X && W && ids && Y, KTMI_EINVAL, "moe_a8_vec: null pointer");
  KTMI_REQUIRE(aligned(W, 16) && aligned(workspace, 16), KTMI_EINVAL, "moe_a8_vec: W and workspace must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  int rc = launch_quantize_q8_1(X, x_dtype, cols, tokens, (uint8_t*)workspace, s);
  if (rc) return rc;
  const int64_t rb = row_bytes(cols, ggml_type);
  return launch_moe_gemv((const uint8_t*)workspace, q8_1_row_bytes(cols), W, w_is_table, rows * rb, ids, top_k,
                         tokens * top_k, ggml_type, rows, cols, Y, x_dtype, per_route, 0x7FFFFFFF, s);
}

int ktmi_dequant_experts(const void* raw, int64_t raw_stride, int ggml_type, int64_t n, int64_t rows, int64_t cols,
                         void* out_bf16, int64_t out_stride, void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(type_ok(ggml_type), KTMI_ETYPE, "dequant: no GPU dequantizer for ggml type %d", ggml_type);
  KTMI_REQUIRE(n >= 0 && rows >= 0 && cols > 0 && cols % blck_size(ggml_type) == 0, KTMI_EINVAL,
               "dequant: n %lld rows %lld cols %lld (block %lld)", (long long)n, (long long)rows, (long long)cols,
               (long long)blck_size(ggml_type));
  KTMI_REQUIRE(n <= 65535, KTMI_EINVAL, "dequant: %lld experts per call (at most 65535)", (long long)n);
  if (n == 0 || rows == 0) return KTMI_OK;
  KTMI_REQUIRE(raw_stride >= rows * row_bytes(cols, ggml_type) && raw_stride % 2 == 0, KTMI_EINVAL,
               "dequant: raw_stride %lld (expert bytes %lld, must be even)", (long long)raw_stride,
               (long long)(rows * row_bytes(cols, ggml_type)));
  KTMI_REQUIRE(out_stride >= rows * cols && out_stride % 8 == 0, KTMI_EINVAL,
               "dequant: out_stride %lld must be >= rows*cols and a multiple of 8", (long long)out_stride);
  KTMI_REQUIRE(raw && out_bf16 && aligned(raw, 16) && aligned(out_bf16, 16), KTMI_EINVAL,
               "dequant: raw and out must be 16-byte aligned device pointers");
  KTMI_REQUIRE(ggml_type != GGML_Q4_K || raw_stride % 16 == 0, KTMI_EINVAL, "dequant: Q4_K raw_stride must be a multiple of 16");
  return launch_dequant((const uint8_t*)raw, raw_stride, ggml_type, n, rows, cols, (uint16_t*)out_bf16, out_stride,
                        (hipStream_t)stream);
}

int ktmi_hot_route(const int32_t* ids, int64_t n, const int32_t* log2slot, const int32_t* log2cpu, float* counts,
                   int32_t* slot_ids, int32_t* cpu_ids, void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(n >= 0, KTMI_EINVAL, "hot_route: n %lld", (long long)n);
  if (n == 0) return KTMI_OK;
  KTMI_REQUIRE(ids && log2slot && log2cpu && slot_ids && cpu_ids, KTMI_EINVAL, "hot_route: null pointer");
  return launch_route(ids, n, log2slot, log2cpu, counts, slot_ids, cpu_ids, (hipStream_t)stream);
}

int ktmi_silu_and_mul(const void* h, int dtype, int64_t R, int64_t N, void* out, void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(dtype_ok(dtype), KTMI_EINVAL, "silu_and_mul: dtype %d", dtype);
  KTMI_REQUIRE(R >= 0 && N > 0, KTMI_EINVAL, "silu_and_mul: R %lld N %lld", (long long)R, (long long)N);
  if (R == 0) return KTMI_OK;
  KTMI_REQUIRE(h && out, KTMI_EINVAL, "silu_and_mul: null pointer");
  return launch_silu_and_mul(h, dtype, R, N, out, (hipStream_t)stream);
}

int ktmi_combine(const void* out, int dtype, const float* w, int64_t T, int64_t top_k, int64_t K, void* res,
                 void* stream) {
  g_err[0] = 0;
  KTMI_REQUIRE(dtype_ok(dtype), KTMI_EINVAL, "combine: dtype %d", dtype);
  KTMI_REQUIRE(T >= 0 && top_k > 0 && K > 0, KTMI_EINVAL, "combine: T %lld top_k %lld K %lld", (long long)T,
               (long long)top_k, (long long)K);
  if (T == 0) return KTMI_OK;
  KTMI_REQUIRE(out && w && res, KTMI_EINVAL, "combine: null pointer");
  return launch_combine(out, dtype, w, T, top_k, K, res, (hipStream_t)stream);
}

// ---- scratch for ktmi_moe_layer_noalloc
// A file-scope device array that stands in for the caller's workspace. In host code its
// name is a host-side stand-in, not a device address: the address on each device comes
// from hipGetSymbolAddress, taken once per device with that device current, and only that
// address is ever handed to kernels. Each GPU holds its own copy until the process ends.
static __device__ __align__(256) uint8_t scratch[KTMI_NOALLOC_SCRATCH_BYTES];
static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

static int scratch_of_current_device(void** out) {
  int dev = 0;
  KTMI_HIP_TRY(hipGetDevice(&dev));
  KTMI_REQUIRE(dev >= 0 && dev < kMaxDevices, KTMI_EINVAL, "moe_layer_noalloc: device %d (at most %d)", dev,
               kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    KTMI_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    KTMI_REQUIRE(p != nullptr, KTMI_EHIP, "moe_layer_noalloc: no device address for the scratch array on device %d",
                 dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KTMI_OK;
}

// Below 64 routes the GEMV mode's two launches match or beat the decode mode's three
// (graph-replayed steps of the 2048 x 512 Q4_K layer with 32 hot slots: 13.0 against 15.0 us at
// 8 routes, 19.5 against 19.2 at 32); from 64 routes the decode mode's MFMAs win (23.0 against
// 25.8 at 64, 24.2 against 30.9 at 128).
constexpr int64_t kDecodeMinRoutes = 64;

int ktmi_moe_layer_mode(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  if (tokens * top_k > kGemvMaxRoutes) return KTMI_MODE_GROUPED;
  return L && tokens * top_k >= kDecodeMinRoutes && decode_mfma_fits(L, tokens, top_k) ? KTMI_MODE_DECODE
                                                                                       : KTMI_MODE_GEMV;
}

static int64_t gemv_layer_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k) {
  // q8_1(x) | h13 bf16 [R, 2N] | h bf16 [R, N] | q8_1(h) | out bf16 [R, K]
  const int64_t R = tokens * top_k;
  auto al = [](int64_t v) { return (v + 255) & ~(int64_t)255; };
  return al(q8_1_row_bytes(L->hidden) * tokens) + al(R * 2 * L->inter * 2) + al(R * L->inter * 2) +
         al(q8_1_row_bytes(L->inter) * R) + al(R * L->hidden * 2);
}

static int check_layer(const ktmi_layer* L) {
  KTMI_REQUIRE(L, KTMI_EINVAL, "moe_layer: null layer");
  KTMI_REQUIRE(type_ok(L->type13) && type_ok(L->type2), KTMI_ETYPE, "moe_layer: ggml types %d/%d", L->type13, L->type2);
  KTMI_REQUIRE(L->hidden > 0 && L->inter > 0 && L->n_slots > 0, KTMI_EINVAL, "moe_layer: hidden %lld inter %lld slots %lld",
               (long long)L->hidden, (long long)L->inter, (long long)L->n_slots);
  KTMI_REQUIRE(L->hidden % blck_size(L->type13) == 0 && L->inter % blck_size(L->type2) == 0, KTMI_EINVAL,
               "moe_layer: hidden %lld / inter %lld not multiples of the block sizes", (long long)L->hidden,
               (long long)L->inter);
  KTMI_REQUIRE(L->w13 && L->w2 && aligned(L->w13, 16) && aligned(L->w2, 16), KTMI_EINVAL,
               "moe_layer: weights must be 16-byte aligned device pointers");
  return KTMI_OK;
}

// Tokens per pass of the grouped mode. Its kernels address x [T, K], H [R, N] and Y [R, K]
// (bf16, R = T top_k) with 32-bit buffer offsets, and an offset at 0xFFFFFFF0 marks a store
// to drop; a pass keeps every one of them under 4 GiB - 64 KiB. A token's output depends only
// on its own routes, so a longer layer runs as consecutive passes over token slices, each
// with the whole workspace.
static int64_t grouped_pass_tokens(const ktmi_layer* L, int64_t top_k) {
  const int64_t limit = 0xFFFF0000ll;
  const int64_t per_token = 2 * top_k * (L->hidden > L->inter ? L->hidden : L->inter);
  const int64_t t = limit / per_token;
  return t >= 256 ? t / 256 * 256 : (t > 0 ? t : 1);
}

int64_t ktmi_moe_layer_pass_tokens(const ktmi_layer* L, int64_t top_k) {
  if (!L || top_k <= 0 || L->hidden <= 0 || L->inter <= 0) return 0;
  return grouped_pass_tokens(L, top_k);
}

int64_t ktmi_moe_layer_workspace(const ktmi_layer* L, int64_t tokens, int64_t top_k, int mode) {
  if (!L || tokens < 0 || top_k <= 0) return 0;
  if (mode == KTMI_MODE_AUTO) mode = ktmi_moe_layer_mode(L, tokens, top_k);
  if (mode == KTMI_MODE_DECODE) return decode_mfma_fits(L, tokens, top_k) ? decode_mfma_workspace(L, tokens, top_k) : 0;
  if (mode == KTMI_MODE_GEMV)
    return decode_layer_fits(L, tokens, top_k) ? decode_layer_workspace(L, tokens, top_k)
                                               : gemv_layer_workspace(L, tokens, top_k);
  const int64_t pass = grouped_pass_tokens(L, top_k);
  return grouped_plan(tokens < pass ? tokens : pass, top_k, L->n_slots, L->hidden, L->inter).total;
}

int ktmi_moe_layer(const ktmi_layer* L, const void* x, const float* topk_w, const int32_t* slot_ids, int64_t tokens,
                   int64_t top_k, void* y, void* workspace, int64_t ws_bytes, int mode, void* stream) {
  g_err[0] = 0;
  int rc = check_layer(L);
  if (rc) return rc;
  KTMI_REQUIRE(tokens >= 0 && top_k > 0, KTMI_EINVAL, "moe_layer: tokens %lld top_k %lld", (long long)tokens,
               (long long)top_k);
  if (tokens == 0) return KTMI_OK;
  KTMI_REQUIRE(x && topk_w && slot_ids && y && workspace, KTMI_EINVAL, "moe_layer: null pointer");
  KTMI_REQUIRE(aligned(x, 16) && aligned(y, 16) && aligned(workspace, 256), KTMI_EINVAL,
               "moe_layer: x, y 16-byte and workspace 256-byte aligned");
  if (mode == KTMI_MODE_AUTO) mode = ktmi_moe_layer_mode(L, tokens, top_k);
  const int64_t need = ktmi_moe_layer_workspace(L, tokens, top_k, mode);
  KTMI_REQUIRE(ws_bytes >= need, KTMI_ESPACE, "moe_layer: workspace %lld < %lld bytes", (long long)ws_bytes,
               (long long)need);
  hipStream_t s = (hipStream_t)stream;
  const int64_t R = tokens * top_k;
  const int64_t K = L->hidden, N = L->inter;
  if (mode == KTMI_MODE_DECODE) {
    KTMI_REQUIRE(decode_mfma_fits(L, tokens, top_k), KTMI_EINVAL,
                 "moe_layer: the decode mode takes at most %d routes of %d tokens, at most 512 slots, hidden and "
                 "intermediate sizes that are multiples of 256, and rows that fit its staging (16 gate and 16 up "
                 "rows in %d bytes, 16 down rows in %d bytes)",
                 DM_MAX_ROUTES, DM_MAX_TOKENS, DM_GU_LDS, DM_DOWN_WAVE_LDS);
    return launch_decode_mfma(L, (const uint16_t*)x, topk_w, slot_ids, tokens, top_k, (uint16_t*)y, (uint8_t*)workspace,
                              s);
  }
  if (mode == KTMI_MODE_GEMV && decode_layer_fits(L, tokens, top_k))
    return launch_decode_layer(L, (const uint16_t*)x, topk_w, slot_ids, tokens, top_k, (uint16_t*)y,
                               (uint8_t*)workspace, s);
  if (mode == KTMI_MODE_GEMV) {
    KTMI_REQUIRE(R <= 65535, KTMI_EINVAL, "moe_layer: GEMV mode takes at most 65535 routes");
    auto al = [](int64_t v) { return (v + 255) & ~(int64_t)255; };
    uint8_t* p = (uint8_t*)workspace;
    uint8_t* xq = p; p += al(q8_1_row_bytes(K) * tokens);
    uint16_t* h13 = (uint16_t*)p; p += al(R * 2 * N * 2);
    uint16_t* h = (uint16_t*)p; p += al(R * N * 2);
    uint8_t* hq = p; p += al(q8_1_row_bytes(N) * R);
    uint16_t* out = (uint16_t*)p;
    // the slot ids are the per-route expert ids of the GEMV (cold = -1)
    record_stage(0, s);
    rc = launch_quantize_q8_1(x, KTMI_BF16, K, tokens, xq, s);
    if (rc) return rc;
    record_stage(1, s);
    rc = launch_moe_gemv(xq, q8_1_row_bytes(K), L->w13, L->w_is_table, 2 * N * row_bytes(K, L->type13), slot_ids,
                         top_k, R, L->type13, 2 * N, K, h13, KTMI_BF16, 0, (int)L->n_slots, s);
    if (rc) return rc;
    record_stage(2, s);
    rc = launch_silu_and_mul(h13, KTMI_BF16, R, N, h, s);
    if (rc) return rc;
    rc = launch_quantize_q8_1(h, KTMI_BF16, N, R, hq, s);
    if (rc) return rc;
    record_stage(3, s);
    rc = launch_moe_gemv(hq, q8_1_row_bytes(N), L->w2, L->w_is_table, K * row_bytes(N, L->type2), slot_ids, 1, R,
                         L->type2, K, N, out, KTMI_BF16, 0, (int)L->n_slots, s);
    if (rc) return rc;
    record_stage(4, s);
    rc = launch_combine(out, KTMI_BF16, topk_w, tokens, top_k, K, y, s);
    record_stage(5, s);
    return rc;
  }
  KTMI_REQUIRE(mode == KTMI_MODE_GROUPED, KTMI_EINVAL, "moe_layer: mode %d", mode);
  const int64_t pass = grouped_pass_tokens(L, top_k);
  for (int64_t t0 = 0; t0 < tokens; t0 += pass) {
    const int64_t nt = tokens - t0 < pass ? tokens - t0 : pass;
    const GroupedPlan P = grouped_plan(nt, top_k, L->n_slots, K, N);
    rc = launch_grouped_layer(L, (const uint16_t*)x + t0 * K, topk_w + t0 * top_k, slot_ids + t0 * top_k, nt, top_k,
                              (uint16_t*)y + t0 * K, (uint8_t*)workspace, P, s);
    if (rc) return rc;
  }
  return KTMI_OK;
}

int ktmi_moe_layer_noalloc(const ktmi_layer* L, const void* x, const float* topk_w, const int32_t* slot_ids,
                           int64_t tokens, int64_t top_k, void* y, int mode, void* stream) {
  g_err[0] = 0;
  int rc = check_layer(L);
  if (rc) return rc;
  KTMI_REQUIRE(tokens >= 0 && top_k > 0, KTMI_EINVAL, "moe_layer_noalloc: tokens %lld top_k %lld", (long long)tokens,
               (long long)top_k);
  if (tokens == 0) return KTMI_OK;
  if (mode == KTMI_MODE_AUTO) mode = ktmi_moe_layer_mode(L, tokens, top_k);
  const int64_t need = ktmi_moe_layer_workspace(L, tokens, top_k, mode);
  KTMI_REQUIRE(need <= KTMI_NOALLOC_SCRATCH_BYTES, KTMI_ESPACE,
               "moe_layer_noalloc: %lld tokens x top-%lld need %lld bytes of scratch, more than the %lld bytes the "
               "library holds per GPU (call ktmi_moe_layer with a workspace instead)",
               (long long)tokens, (long long)top_k, (long long)need, (long long)KTMI_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc) return rc;
  return ktmi_moe_layer(L, x, topk_w, slot_ids, tokens, top_k, y, ws, KTMI_NOALLOC_SCRATCH_BYTES, mode, stream);
}

}  // extern "C"
