// The CPU expert engine's internal interface (cpu_moe.cpp), used by the C-ABI and the
// GPU <-> CPU handoff in handoff.hip.
#pragma once
#include <stdint.h>

namespace ktmi_cpu {

struct Engine;

// Expert banks: gate / up uint8 [E, N rows x row_bytes(K, type13)], down uint8
// [E, K rows x row_bytes(N, type2)] in host memory, kept alive by the caller.
// threads <= 0: min(16, hardware threads) - 1 (one left to the thread driving the GPU). Returns nullptr (and a message) on bad input.
Engine* engine_create(int64_t hidden, int64_t inter, int64_t n_experts, int type13, int type2, const uint8_t* gate,
                      const uint8_t* up, const uint8_t* down, int threads, const char** err);
void engine_destroy(Engine* e);
// out bf16 [T, hidden] = bf16(sum over k of w[t, k] * FFN_{ids[t, k]}(x[t])) in route order;
// ids outside [0, n_experts) add nothing. 0 or -1 (allocation failure).
int engine_forward(Engine* e, int64_t T, int64_t top_k, const int32_t* ids, const float* w, const uint16_t* x,
                   uint16_t* out);
int engine_threads(const Engine* e);
// "avx512-vnni" or "scalar": the engine's integer dot-product kernels (AVX-512 VNNI when
// the host has it, unless KTMI_CPU_ISA=scalar was set when the engine was created)
const char* engine_isa(const Engine* e);

}  // namespace ktmi_cpu
