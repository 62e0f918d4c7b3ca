// Layer-weight streamer: experts' raw GGUF bytes move from pinned host banks into
// double-buffered device slots on a copy stream while the compute stream works on the
// other slot (the reference's KTStreamPrefillGGUF: _Slot with dma_done / compute_done
// events, _stage and the group loop of run, P:40543-40550, 40773-40787, 40928-40992).
//
// A slot holds a group of up to max_group experts in the layout the grouped kernels read
// directly: w13 [n, 2N rows, row bytes] (gate rows then up rows of each expert) and
// w2 [n, K rows, row bytes]. Staging a group is three copies on the copy stream: the gate
// and up parts of the bank rows [first, first+n) scattered into the slot's w13 with a 2D
// copy each (destination pitch = one expert's gate+up bytes), and the down part as one
// contiguous copy. No bf16 copy of the weights is made: the grouped GEMM dequantises the
// raw blocks as it goes (the reference dequantises every group into bf16 buffers first,
// P:40789-40798).
//
// Ordering: stage(slot) makes the copy stream wait for the slot's `released` event (set by
// release() on the compute stream after the last kernel that read the slot) before its
// copies, then records `loaded`; acquire(slot) makes the compute stream wait for `loaded`.
// All streams keep the default priority.
#include "kernels.h"

struct ktmi_streamer {
  int device;
  int64_t max_group, part13, part2;  // experts per slot; bytes per expert of w13 and w2
  int n_slots;
  uint8_t* w13[KTMI_STREAM_MAX_SLOTS];
  uint8_t* w2[KTMI_STREAM_MAX_SLOTS];
  hipEvent_t loaded[KTMI_STREAM_MAX_SLOTS];
  hipEvent_t released[KTMI_STREAM_MAX_SLOTS];
  bool used[KTMI_STREAM_MAX_SLOTS];  // released has been recorded at least once
  hipStream_t copy;
};

namespace ktmi {
namespace {

__global__ void remap_ids_kernel(const int32_t* __restrict__ ids, int64_t n, int32_t base, int32_t count,
                                 int32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t e = ids[i];
  out[i] = (e >= base && e < base + count) ? e - base : -1;
}

// acc[i] = bf16(float(acc[i]) + float(x[i])), 8 values per thread
__global__ void add_bf16_kernel(uint16_t* __restrict__ acc, const uint16_t* __restrict__ x, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i + 8 <= n) {
    u32x4_t a = *(const u32x4_t*)(acc + i);
    const u32x4_t b = *(const u32x4_t*)(x + i);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      a[k] = f2bf2(bf2f(a[k] & 0xFFFF) + bf2f(b[k] & 0xFFFF), bf2f(a[k] >> 16) + bf2f(b[k] >> 16));
    *(u32x4_t*)(acc + i) = a;
  } else {
    for (int64_t j = i; j < n; ++j) acc[j] = f2bf(bf2f(acc[j]) + bf2f(x[j]));
  }
}

void destroy(ktmi_streamer* s) {
  if (!s) return;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(s->device);
  if (s->copy) (void)hipStreamSynchronize(s->copy);
  for (int i = 0; i < s->n_slots; ++i) {
    // the compute stream's last group on this slot may still be reading it
    if (s->released[i]) (void)hipEventSynchronize(s->released[i]);
    if (s->loaded[i]) (void)hipEventDestroy(s->loaded[i]);
    if (s->released[i]) (void)hipEventDestroy(s->released[i]);
    if (s->w13[i]) (void)hipFree(s->w13[i]);
    if (s->w2[i]) (void)hipFree(s->w2[i]);
  }
  if (s->copy) (void)hipStreamDestroy(s->copy);
  (void)hipSetDevice(prev);
  delete s;
}

}  // namespace
}  // namespace ktmi

using namespace ktmi;

extern "C" {

ktmi_streamer* ktmi_streamer_create(int64_t max_group, int64_t part13, int64_t part2, int n_slots) {
  clear_error();
  if (max_group <= 0 || part13 <= 0 || part2 <= 0 || n_slots < 2 || n_slots > KTMI_STREAM_MAX_SLOTS) {
    set_error("streamer_create: max_group %lld, part bytes %lld/%lld, slots %d (2..%d)", (long long)max_group,
              (long long)part13, (long long)part2, n_slots, KTMI_STREAM_MAX_SLOTS);
    return nullptr;
  }
  ktmi_streamer* s = new ktmi_streamer{};
  s->max_group = max_group;
  s->part13 = part13;
  s->part2 = part2;
  s->n_slots = n_slots;
  hipError_t e = hipGetDevice(&s->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s->copy, hipStreamNonBlocking);
  for (int i = 0; i < n_slots && e == hipSuccess; ++i) {
    e = hipMalloc((void**)&s->w13[i], (size_t)(max_group * part13));
    if (e == hipSuccess) e = hipMalloc((void**)&s->w2[i], (size_t)(max_group * part2));
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s->loaded[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s->released[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    set_error("streamer_create: %s", hipGetErrorString(e));
    destroy(s);
    return nullptr;
  }
  return s;
}

int ktmi_streamer_destroy(ktmi_streamer* s) {
  clear_error();
  destroy(s);
  return KTMI_OK;
}

int ktmi_streamer_slot(ktmi_streamer* s, int slot, void** w13, void** w2) {
  clear_error();
  KTMI_REQUIRE(s && slot >= 0 && slot < s->n_slots, KTMI_EINVAL, "streamer_slot: slot %d", slot);
  if (w13) *w13 = s->w13[slot];
  if (w2) *w2 = s->w2[slot];
  return KTMI_OK;
}

int ktmi_streamer_stage(ktmi_streamer* s, int slot, const ktmi_bank* bank, int64_t first, int64_t n) {
  clear_error();
  KTMI_REQUIRE(s && bank && slot >= 0 && slot < s->n_slots, KTMI_EINVAL, "streamer_stage: slot %d", slot);
  KTMI_REQUIRE(n >= 1 && n <= s->max_group && first >= 0 && first + n <= bank->n_experts, KTMI_EINVAL,
               "streamer_stage: experts [%lld, %lld) of %lld, group of at most %lld", (long long)first,
               (long long)(first + n), (long long)bank->n_experts, (long long)s->max_group);
  KTMI_REQUIRE(bank->part_gate > 0 && bank->part_up == bank->part_gate &&
                   bank->part_gate + bank->part_up <= s->part13 && bank->part_down > 0 &&
                   bank->part_down <= s->part2,
               KTMI_EINVAL, "streamer_stage: part bytes %lld/%lld/%lld vs slot %lld/%lld", (long long)bank->part_gate,
               (long long)bank->part_up, (long long)bank->part_down, (long long)s->part13, (long long)s->part2);
  KTMI_REQUIRE(bank->gate && bank->up && bank->down, KTMI_EINVAL, "streamer_stage: null bank pointer");
  const int64_t pg = bank->part_gate, pd = bank->part_down;
  const int64_t stride13 = 2 * pg;  // slot w13 expert stride: [gate; up] rows back to back
  if (s->used[slot]) KTMI_HIP_TRY(hipStreamWaitEvent(s->copy, s->released[slot], 0));
  const uint8_t* gate = (const uint8_t*)bank->gate + first * pg;
  const uint8_t* up = (const uint8_t*)bank->up + first * pg;
  const uint8_t* down = (const uint8_t*)bank->down + first * pd;
  KTMI_HIP_TRY(hipMemcpy2DAsync(s->w13[slot], (size_t)stride13, gate, (size_t)pg, (size_t)pg, (size_t)n,
                                hipMemcpyHostToDevice, s->copy));
  KTMI_HIP_TRY(hipMemcpy2DAsync(s->w13[slot] + pg, (size_t)stride13, up, (size_t)pg, (size_t)pg, (size_t)n,
                                hipMemcpyHostToDevice, s->copy));
  KTMI_HIP_TRY(hipMemcpyAsync(s->w2[slot], down, (size_t)(n * pd), hipMemcpyHostToDevice, s->copy));
  KTMI_HIP_TRY(hipEventRecord(s->loaded[slot], s->copy));
  return KTMI_OK;
}

int ktmi_streamer_acquire(ktmi_streamer* s, int slot, void* stream) {
  clear_error();
  KTMI_REQUIRE(s && slot >= 0 && slot < s->n_slots, KTMI_EINVAL, "streamer_acquire: slot %d", slot);
  KTMI_HIP_TRY(hipStreamWaitEvent((hipStream_t)stream, s->loaded[slot], 0));
  return KTMI_OK;
}

int ktmi_streamer_release(ktmi_streamer* s, int slot, void* stream) {
  clear_error();
  KTMI_REQUIRE(s && slot >= 0 && slot < s->n_slots, KTMI_EINVAL, "streamer_release: slot %d", slot);
  KTMI_HIP_TRY(hipEventRecord(s->released[slot], (hipStream_t)stream));
  s->used[slot] = true;
  return KTMI_OK;
}

void* ktmi_streamer_copy_stream(ktmi_streamer* s) { return s ? (void*)s->copy : nullptr; }

int ktmi_streamer_sync(ktmi_streamer* s) {
  clear_error();
  KTMI_REQUIRE(s, KTMI_EINVAL, "streamer_sync: null streamer");
  KTMI_HIP_TRY(hipStreamSynchronize(s->copy));
  return KTMI_OK;
}

int ktmi_remap_ids(const int32_t* ids, int64_t n, int32_t base, int32_t count, int32_t* out, void* stream) {
  clear_error();
  KTMI_REQUIRE(n >= 0 && count >= 0, KTMI_EINVAL, "remap_ids: n %lld count %d", (long long)n, count);
  if (n == 0) return KTMI_OK;
  KTMI_REQUIRE(ids && out, KTMI_EINVAL, "remap_ids: null pointer");
  remap_ids_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(ids, n, base, count, out);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

int ktmi_add_bf16(void* acc, const void* x, int64_t n, void* stream) {
  clear_error();
  KTMI_REQUIRE(n >= 0, KTMI_EINVAL, "add_bf16: n %lld", (long long)n);
  if (n == 0) return KTMI_OK;
  KTMI_REQUIRE(acc && x && ((uintptr_t)acc % 16) == 0 && ((uintptr_t)x % 16) == 0, KTMI_EINVAL,
               "add_bf16: null or not 16-byte aligned");
  const int64_t threads = (n + 7) / 8;
  add_bf16_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, (hipStream_t)stream>>>((uint16_t*)acc,
                                                                                     (const uint16_t*)x, n);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

void* ktmi_host_alloc(int64_t bytes) {
  clear_error();
  if (bytes <= 0) {
    set_error("host_alloc: %lld bytes", (long long)bytes);
    return nullptr;
  }
  void* p = nullptr;
  const hipError_t e = hipHostMalloc(&p, (size_t)bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    set_error("host_alloc: %s", hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

int ktmi_host_free(void* p) {
  clear_error();
  if (p) KTMI_HIP_TRY(hipHostFree(p));
  return KTMI_OK;
}

}  // extern "C"
