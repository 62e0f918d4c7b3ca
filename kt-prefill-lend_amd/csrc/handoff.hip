// The CPU expert engine behind the C ABI, and the GPU <-> CPU handoff of one MoE layer:
// kt-kernel's submit_forward / sync_forward as KTEPWrapperMethod calls them around the GPU
// method (P:10590-10602) and kt_uva_handoff.submit / sync_add (P:41025-41301).
//
// submit(x, ids, weights) on the compute stream: one kernel writes them into the engine's
// pinned staging buffers through their device addresses (the reference's UVA staging,
// kt_uva_handoff._stage_kernel; one launch instead of three small copies) and publishes the
// submit's sequence number in pinned memory once all its blocks' writes are visible; the
// engine's worker thread spins on that number (an event on the stream is the fallback),
// runs the cold routes on the host cores (cpu_moe.cpp) into a pinned bf16 output.
// The stream goes on with the GPU's hot experts meanwhile. sync_add(out): out = bf16(out +
// cpu) on the stream (the wrapper's `output + cpu_output`), the add kernel reading the CPU
// output from pinned memory through its device address (no separate copy), and the host
// spins until the worker is done, as sync_forward blocks. For decode windows the add is
// enqueued before that wait and starts on a completion word the worker stores in pinned
// memory, so no launch sits between the CPU side's end and the add; larger layers launch
// their add after the wait. The pinned output is written again only after that add has
// completed (event out_free), so back-to-back layers cannot overwrite it early. One submit
// is outstanding at a time per engine.
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>

#include "cpu_moe.h"
#include "kernels.h"

// sync_add enqueues its add ahead of the CPU side's end for layers of at most this many
// tokens (decode windows, whose CPU side takes milliseconds); that add waits at most
// KTMI_WAIT_ADD_US (ktmi_cpu_moe_set_add_wait changes it) for the CPU side. Larger layers
// are added once the CPU side is done.
constexpr int64_t KTMI_WAIT_ADD_MAX_TOKENS = 256;
constexpr int64_t KTMI_WAIT_ADD_US = 10 * 1000 * 1000;

static int64_t host_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

struct ktmi_cpu_moe {
  ktmi_cpu::Engine* eng = nullptr;
  int device = 0;
  int64_t K = 0, max_tokens = 0, max_top_k = 0;
  uint16_t* x_h = nullptr;
  int32_t* ids_h = nullptr;
  float* w_h = nullptr;
  uint16_t* out_h = nullptr;
  uint16_t* x_hd = nullptr;  // device addresses of the pinned staging buffers
  int32_t* ids_hd = nullptr;
  float* w_hd = nullptr;
  uint16_t* out_hd = nullptr;
  // staging handshake: the staging kernel's last block stores the submit's sequence number
  // into pinned memory (seq_h, device address seq_hd) after every block's writes; blocks_d
  // counts the blocks done (device memory, reset by the last block)
  uint32_t* seq_h = nullptr;
  uint32_t* seq_hd = nullptr;
  uint32_t* blocks_d = nullptr;
  uint32_t seq = 0;
  // completion words the worker publishes in pinned memory (device address fin_hd) for the
  // add kernel sync_add enqueues ahead of the CPU side's end: [0] the last finished submit's
  // sequence number, [1] the last successful one, [2] the last one whose add stopped waiting
  uint32_t* fin_h = nullptr;
  uint32_t* fin_hd = nullptr;
  uint64_t wait_ticks = 0;  // that add's wait bound, in wall-clock ticks
  int64_t wait_us = 0;      // the same bound in microseconds
  int wall_khz = 0;         // the GPU wall clock's rate
  // host clock when the worker published the last completion word (after fin[0])
  std::atomic<int64_t> done_ns{0};
  hipEvent_t in_ready = nullptr;
  // out_free[s & 1]: submit s's add is done with the pinned output. Two, so that sync_add of
  // submit s, which may enqueue its add before the worker has started on s, never re-records
  // the event the worker of s waits on (that of submit s - 1).
  hipEvent_t out_free[2] = {nullptr, nullptr};
  bool out_free_pending[2] = {false, false};
  std::thread worker;
  std::mutex m;
  std::condition_variable cv;
  enum State { IDLE, SUBMITTED, DONE };
  std::atomic<int> state{IDLE};
  int64_t T = 0, k = 0;
  int rc = 0;
  std::atomic<bool> stop{false};
};

namespace {

using ktmi::bf2f;
using ktmi::f2bf;
using ktmi::f2bf2;

// x [T, K] bf16 (16-byte chunks), ids and weights [P] into pinned host memory; then the
// last block to finish publishes `seq` in pinned memory: every block makes its writes
// visible to the host (system-scope fence) before it counts itself done, and the block that
// counts last stores seq with system-scope release (and resets the counter for the next
// submit, which the stream orders after this kernel)
__global__ __launch_bounds__(256) void stage_kernel(const u32x4_t* __restrict__ x, int64_t nx,
                                                     const int32_t* __restrict__ ids, const float* __restrict__ w,
                                                     int64_t P, u32x4_t* __restrict__ xh, int32_t* __restrict__ idsh,
                                                     float* __restrict__ wh, uint32_t* blocks_done,
                                                     uint32_t* seq_out, uint32_t seq) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nx; i += stride) xh[i] = x[i];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < P; i += stride) {
    idsh[i] = ids[i];
    wh[i] = w[i];
  }
  __threadfence_system();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t done = atomicAdd(blocks_done, 1u);
    if (done == gridDim.x - 1) {
      __threadfence_system();
      *blocks_done = 0;
      __hip_atomic_store(seq_out, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// out += the CPU output of submit `seq` (add_bf16_kernel's arithmetic), enqueued before the
// CPU side has finished: thread 0 of each block spins on the completion word fin[0] (system
// scope, up to `limit` wall-clock ticks), then the block adds its 8 values a thread. A
// forward that failed (fin[1] != seq) leaves out as it is; a wait past the bound writes NaN
// and records seq in fin[2] for sync_add to report.
__global__ __launch_bounds__(256) void wait_add_kernel(uint16_t* __restrict__ acc, const uint16_t* __restrict__ x,
                                                        int64_t n, uint32_t* fin, uint32_t seq, uint64_t limit) {
  __shared__ int go;
  if (threadIdx.x == 0) {
    const uint64_t t0 = (uint64_t)wall_clock64();
    int st = 0;  // 0: timed out, 1: add, 2: the forward failed
    for (;;) {
      if ((int32_t)(__hip_atomic_load(fin, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) - seq) >= 0) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");
        st = __hip_atomic_load(fin + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == seq ? 1 : 2;
        break;
      }
      if ((uint64_t)wall_clock64() - t0 > limit) break;
      __builtin_amdgcn_s_sleep(4);
    }
    if (st == 0) __hip_atomic_store(fin + 2, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    go = st;
  }
  __syncthreads();
  if (go == 2) return;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i + 8 <= n) {
    u32x4_t a = *(const u32x4_t*)(acc + i);
    if (go == 1) {
      const u32x4_t b = *(const u32x4_t*)(x + i);
#pragma unroll
      for (int k = 0; k < 4; ++k)
        a[k] = f2bf2(bf2f(a[k] & 0xFFFF) + bf2f(b[k] & 0xFFFF), bf2f(a[k] >> 16) + bf2f(b[k] >> 16));
    } else {
      a = u32x4_t{0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u};
    }
    *(u32x4_t*)(acc + i) = a;
  } else {
    for (int64_t j = i; j < n; ++j) acc[j] = go == 1 ? f2bf(bf2f(acc[j]) + bf2f(x[j])) : (uint16_t)0x7FC0;
  }
}

// Wait until pred() holds: spin up to `spin_us` microseconds (a decode layer's handoff is
// tens of microseconds), then sleep on the engine's condition variable.
template <typename Pred>
void wait_for(ktmi_cpu_moe* h, Pred pred, int spin_us) {
  const auto t0 = std::chrono::steady_clock::now();
  for (int i = 0;; ++i) {
    if (pred()) return;
    _mm_pause();
    if ((i & 63) == 63 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us)) break;
  }
  std::unique_lock<std::mutex> g(h->m);
  h->cv.wait(g, pred);
}

// an event wait that polls (a short wait on the stream's staging kernel), then blocks
int event_wait(hipEvent_t e) {
  for (int i = 0; i < 256; ++i) {
    const hipError_t q = hipEventQuery(e);
    if (q == hipSuccess) return 0;
    if (q != hipErrorNotReady) return -2;
    _mm_pause();
  }
  return hipEventSynchronize(e) == hipSuccess ? 0 : -2;
}

// the staged inputs of submit `seq` are in pinned memory: spin on the sequence number the
// staging kernel publishes (no runtime call on the way); past `spin_us` fall back to the
// stream event, which also reports a failed stream instead of waiting for ever
int staged_wait(ktmi_cpu_moe* h, uint32_t seq, int spin_us) {
  const auto t0 = std::chrono::steady_clock::now();
  for (int i = 0;; ++i) {
    if ((int32_t)(__atomic_load_n(h->seq_h, __ATOMIC_ACQUIRE) - seq) >= 0) return 0;
    _mm_pause();
    if ((i & 63) == 63 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(spin_us)) break;
  }
  const int rc = event_wait(h->in_ready);
  if (rc) return rc;
  return (int32_t)(__atomic_load_n(h->seq_h, __ATOMIC_ACQUIRE) - seq) >= 0 ? 0 : -3;
}

void worker_loop(ktmi_cpu_moe* h) {
  (void)hipSetDevice(h->device);
  for (;;) {
    wait_for(h, [h] { return h->stop || h->state.load() == ktmi_cpu_moe::SUBMITTED; }, 50);
    if (h->stop) return;
    int rc = staged_wait(h, h->seq, 2000);
    const int prev = (h->seq - 1) & 1;  // the previous submit's add must be done with out_h
    if (rc == 0 && h->out_free_pending[prev]) rc = event_wait(h->out_free[prev]);
    if (rc == 0) rc = ktmi_cpu::engine_forward(h->eng, h->T, h->k, h->ids_h, h->w_h, h->x_h, h->out_h);
    h->rc = rc;
    // the output's stores before the completion words (an add kernel may be waiting on them)
    if (rc == 0) __atomic_store_n(h->fin_h + 1, h->seq, __ATOMIC_RELEASE);
    __atomic_store_n(h->fin_h, h->seq, __ATOMIC_RELEASE);
    h->done_ns.store(host_ns());
    {
      std::lock_guard<std::mutex> g(h->m);
      h->state.store(ktmi_cpu_moe::DONE);
    }
    h->cv.notify_all();
  }
}

void destroy(ktmi_cpu_moe* h) {
  if (!h) return;
  if (h->worker.joinable()) {
    {
      std::lock_guard<std::mutex> g(h->m);
      h->stop = true;
    }
    h->cv.notify_all();
    h->worker.join();
  }
  if (h->in_ready || h->x_h) (void)hipSetDevice(h->device);
  // the last sync_add's add kernel may still be reading the pinned output
  for (int i = 0; i < 2; ++i)
    if (h->out_free_pending[i]) (void)hipEventSynchronize(h->out_free[i]);
  if (h->in_ready) (void)hipEventDestroy(h->in_ready);
  for (int i = 0; i < 2; ++i)
    if (h->out_free[i]) (void)hipEventDestroy(h->out_free[i]);
  if (h->fin_h) (void)hipHostFree(h->fin_h);
  if (h->x_h) (void)hipHostFree(h->x_h);
  if (h->ids_h) (void)hipHostFree(h->ids_h);
  if (h->w_h) (void)hipHostFree(h->w_h);
  if (h->out_h) (void)hipHostFree(h->out_h);
  if (h->seq_h) (void)hipHostFree(h->seq_h);
  if (h->blocks_d) (void)hipFree(h->blocks_d);
  ktmi_cpu::engine_destroy(h->eng);
  delete h;
}

}  // namespace

using namespace ktmi;

extern "C" {

ktmi_cpu_moe* ktmi_cpu_moe_create(int64_t hidden, int64_t inter, int type13, int type2, const ktmi_bank* bank,
                                  int threads, int64_t max_tokens, int64_t max_top_k) {
  clear_error();
  if (!bank || max_tokens < 0 || max_top_k < 0) {
    set_error("cpu_moe_create: null bank or negative sizes");
    return nullptr;
  }
  const char* err = nullptr;
  ktmi_cpu::Engine* eng = ktmi_cpu::engine_create(hidden, inter, bank->n_experts, type13, type2,
                                                  (const uint8_t*)bank->gate, (const uint8_t*)bank->up,
                                                  (const uint8_t*)bank->down, threads, &err);
  if (!eng) {
    set_error("cpu_moe_create: %s", err ? err : "failed");
    return nullptr;
  }
  const int64_t rb13 = row_bytes(hidden, type13), rb2 = row_bytes(inter, type2);
  if (bank->part_gate != inter * rb13 || bank->part_up != inter * rb13 || bank->part_down != hidden * rb2) {
    set_error("cpu_moe_create: bank part bytes %lld/%lld/%lld, expected %lld/%lld/%lld", (long long)bank->part_gate,
              (long long)bank->part_up, (long long)bank->part_down, (long long)(inter * rb13),
              (long long)(inter * rb13), (long long)(hidden * rb2));
    ktmi_cpu::engine_destroy(eng);
    return nullptr;
  }
  ktmi_cpu_moe* h = new ktmi_cpu_moe{};
  h->eng = eng;
  h->K = hidden;
  h->max_tokens = max_tokens;
  h->max_top_k = max_top_k;
  hipError_t e = hipSuccess;
  if (max_tokens > 0 && max_top_k > 0) {  // a forward-only engine makes no HIP call
    const size_t P = (size_t)(max_tokens * max_top_k);
    e = hipGetDevice(&h->device);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->x_h, (size_t)(max_tokens * hidden) * 2, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->ids_h, P * 4, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->w_h, P * 4, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->out_h, (size_t)(max_tokens * hidden) * 2, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&h->in_ready, hipEventDisableTiming);
    for (int i = 0; i < 2; ++i)
      if (e == hipSuccess) e = hipEventCreateWithFlags(&h->out_free[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->x_hd, h->x_h, 0);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->ids_hd, h->ids_h, 0);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->w_hd, h->w_h, 0);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->out_hd, h->out_h, 0);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->seq_h, 64, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->seq_hd, h->seq_h, 0);
    if (e == hipSuccess) e = hipMalloc((void**)&h->blocks_d, 4);
    if (e == hipSuccess) e = hipMemset(h->blocks_d, 0, 4);
    if (e == hipSuccess) e = hipHostMalloc((void**)&h->fin_h, 64, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&h->fin_hd, h->fin_h, 0);
    int khz = 0;
    if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, h->device);
    h->wall_khz = khz > 0 ? khz : 100000;
    h->wait_us = KTMI_WAIT_ADD_US;
    h->wait_ticks = (uint64_t)h->wall_khz * (uint64_t)h->wait_us / 1000ull;
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) {
      __atomic_store_n(h->seq_h, 0u, __ATOMIC_RELEASE);
      for (int i = 0; i < 3; ++i) __atomic_store_n(h->fin_h + i, 0u, __ATOMIC_RELEASE);
    }
  }
  if (e != hipSuccess) {
    set_error("cpu_moe_create: %s", hipGetErrorString(e));
    destroy(h);
    return nullptr;
  }
  if (max_tokens > 0 && max_top_k > 0) h->worker = std::thread(worker_loop, h);
  return h;
}

int ktmi_cpu_moe_destroy(ktmi_cpu_moe* h) {
  clear_error();
  destroy(h);
  return KTMI_OK;
}

int ktmi_cpu_moe_threads(const ktmi_cpu_moe* h) { return h ? ktmi_cpu::engine_threads(h->eng) : 0; }

int ktmi_cpu_moe_set_add_wait(ktmi_cpu_moe* h, int64_t microseconds) {
  clear_error();
  KTMI_REQUIRE(h && h->fin_h, KTMI_EINVAL, "cpu_moe_set_add_wait: no engine with a handoff");
  KTMI_REQUIRE(microseconds >= 1 && microseconds <= 3600ll * 1000 * 1000, KTMI_EINVAL,
               "cpu_moe_set_add_wait: %lld us (1 us .. 1 h)", (long long)microseconds);
  std::lock_guard<std::mutex> g(h->m);
  KTMI_REQUIRE(h->state == ktmi_cpu_moe::IDLE, KTMI_EINVAL, "cpu_moe_set_add_wait: a submitted layer is not synced");
  h->wait_us = microseconds;
  h->wait_ticks = (uint64_t)h->wall_khz * (uint64_t)microseconds / 1000ull;
  return KTMI_OK;
}

const char* ktmi_cpu_moe_isa(const ktmi_cpu_moe* h) { return h ? ktmi_cpu::engine_isa(h->eng) : ""; }

int ktmi_cpu_moe_forward(ktmi_cpu_moe* h, int64_t tokens, int64_t top_k, const int32_t* expert_ids,
                         const float* weights, const void* x_bf16, void* out_bf16) {
  clear_error();
  KTMI_REQUIRE(h && tokens >= 0 && top_k >= 1, KTMI_EINVAL, "cpu_moe_forward: tokens %lld top_k %lld",
               (long long)tokens, (long long)top_k);
  if (tokens == 0) return KTMI_OK;
  KTMI_REQUIRE(expert_ids && weights && x_bf16 && out_bf16, KTMI_EINVAL, "cpu_moe_forward: null pointer");
  {
    std::lock_guard<std::mutex> g(h->m);
    KTMI_REQUIRE(h->state == ktmi_cpu_moe::IDLE, KTMI_EINVAL, "cpu_moe_forward: a submitted layer is not synced");
  }
  const int rc = ktmi_cpu::engine_forward(h->eng, tokens, top_k, expert_ids, weights, (const uint16_t*)x_bf16,
                                          (uint16_t*)out_bf16);
  KTMI_REQUIRE(rc == 0, KTMI_ESPACE, "cpu_moe_forward: out of host memory");
  return KTMI_OK;
}

int ktmi_cpu_moe_submit(ktmi_cpu_moe* h, const void* x_bf16, const int32_t* expert_ids, const float* weights,
                        int64_t tokens, int64_t top_k, void* stream) {
  clear_error();
  KTMI_REQUIRE(h && tokens >= 0 && top_k >= 1, KTMI_EINVAL, "cpu_moe_submit: tokens %lld top_k %lld",
               (long long)tokens, (long long)top_k);
  KTMI_REQUIRE(tokens <= h->max_tokens && top_k <= h->max_top_k, KTMI_EINVAL,
               "cpu_moe_submit: %lld tokens x top-%lld beyond the staging of %lld x %lld", (long long)tokens,
               (long long)top_k, (long long)h->max_tokens, (long long)h->max_top_k);
  std::unique_lock<std::mutex> g(h->m);
  KTMI_REQUIRE(h->state == ktmi_cpu_moe::IDLE, KTMI_EINVAL, "cpu_moe_submit: the previous layer is not synced");
  h->T = tokens;
  h->k = top_k;
  if (tokens == 0) {
    h->rc = 0;
    h->state = ktmi_cpu_moe::DONE;
    return KTMI_OK;
  }
  KTMI_REQUIRE(x_bf16 && expert_ids && weights && ((uintptr_t)x_bf16 % 16) == 0, KTMI_EINVAL,
               "cpu_moe_submit: null pointer or x not 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int64_t nx = tokens * h->K / 8, P = tokens * top_k;  // K is a multiple of 256
  const int64_t blocks = std::min<int64_t>(((nx > P ? nx : P) + 255) / 256, 1024);
  h->seq += 1;
  stage_kernel<<<(unsigned)blocks, 256, 0, s>>>((const u32x4_t*)x_bf16, nx, expert_ids, weights, P,
                                                (u32x4_t*)h->x_hd, h->ids_hd, h->w_hd, h->blocks_d, h->seq_hd,
                                                h->seq);
  KTMI_HIP_TRY(hipGetLastError());
  KTMI_HIP_TRY(hipEventRecord(h->in_ready, s));
  h->state = ktmi_cpu_moe::SUBMITTED;
  g.unlock();
  h->cv.notify_all();
  return KTMI_OK;
}

int ktmi_cpu_moe_sync_add(ktmi_cpu_moe* h, void* out_bf16, void* stream) {
  clear_error();
  KTMI_REQUIRE(h, KTMI_EINVAL, "cpu_moe_sync_add: null engine");
  KTMI_REQUIRE(h->state.load() != ktmi_cpu_moe::IDLE, KTMI_EINVAL, "cpu_moe_sync_add: nothing submitted");
  const int64_t T = h->T;
  const uint32_t seq = h->seq;
  const bool out_ok = out_bf16 && ((uintptr_t)out_bf16 % 16) == 0;
  // the add reads the CPU result straight from pinned memory (no copy to the device first);
  // out_free[seq & 1] marks when it is done, before the worker may write the next result
  // there. A decode window's add goes on the stream now and waits there for the worker's
  // completion word.
  const bool ahead = T > 0 && T <= KTMI_WAIT_ADD_MAX_TOKENS && out_ok;
  hipError_t early = hipSuccess;
  const int64_t enq_ns = host_ns();  // the add's blocks start after this
  if (ahead) {
    const int64_t n = T * h->K;
    wait_add_kernel<<<(unsigned)(((n + 7) / 8 + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        (uint16_t*)out_bf16, h->out_hd, n, h->fin_hd, seq, h->wait_ticks);
    early = hipGetLastError();
    if (early == hipSuccess) early = hipEventRecord(h->out_free[seq & 1], (hipStream_t)stream);
    if (early == hipSuccess) h->out_free_pending[seq & 1] = true;
  }
  // the caller has nothing else to do here: spin through the CPU side's whole duration
  // (a decode layer's is well under this) rather than pay a wake-up on top of it
  wait_for(h, [h] { return h->state.load() == ktmi_cpu_moe::DONE; }, 2000);
  {
    std::lock_guard<std::mutex> g(h->m);
    h->state.store(ktmi_cpu_moe::IDLE);
  }
  KTMI_HIP_TRY(early);
  KTMI_REQUIRE(h->rc == 0, KTMI_EHIP, "cpu_moe_sync_add: the CPU side failed (%d)", h->rc);
  if (T == 0) return KTMI_OK;
  KTMI_REQUIRE(out_ok, KTMI_EINVAL, "cpu_moe_sync_add: output null or not 16-byte aligned");
  if (ahead) {
    // Did any block of the add give up? Each block starts its bound after enq_ns and sees
    // the completion word within microseconds of the worker's store (done_ns): a worker
    // done less than half a bound of at least 1 ms after enq_ns leaves every block time to
    // spare, and no block gave up. Otherwise the blocks' outcome is read once the add has
    // finished: a block that gives up records it in fin[2] before it exits, so a block
    // still deciding cannot be missed.
    const int64_t done_after_us = (h->done_ns.load() - enq_ns) / 1000;
    if (!(h->wait_us >= 1000 && done_after_us < h->wait_us / 2)) {
      KTMI_HIP_TRY(hipEventSynchronize(h->out_free[seq & 1]));
      KTMI_REQUIRE(__atomic_load_n(h->fin_h + 2, __ATOMIC_ACQUIRE) != seq, KTMI_EHIP,
                   "cpu_moe_sync_add: the add stopped waiting for the CPU side after %lld us (its rows are NaN)",
                   (long long)h->wait_us);
    }
    return KTMI_OK;
  }
  const int rc = ktmi_add_bf16(out_bf16, h->out_hd, T * h->K, stream);
  if (rc) return rc;
  KTMI_HIP_TRY(hipEventRecord(h->out_free[seq & 1], (hipStream_t)stream));
  h->out_free_pending[seq & 1] = true;
  return KTMI_OK;
}

}  // extern "C"
