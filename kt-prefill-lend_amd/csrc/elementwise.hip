// Memory-bound kernels of the hot-expert path: GGUF dequantisation to bf16 (through the
// grouped GEMMs' decoder), the hot
// cache's route lookup, q8_1 activation quantisation, SiLU*mul and the weighted top-k
// combine.
#include "bpiece.h"
#include "kernels.h"

namespace ktmi {

// ---------------------------------------------------------------- dequant
// The grouped GEMMs' own decoder (bpiece.h) run stand-alone, so the bytes-to-bf16 step the
// GEMMs feed to the matrix cores is the one this entry point exposes (and its tests pin):
// the same lane -> (row, half) map (lane % 32 = row of a 32-row group, lane / 32 = half h
// of a 64-value step), the same load_head / load<SUB> / decode<SUB> calls. Each wave runs
// 32 rows over the 4 steps of one 256-value super-block column and writes every decoded
// 8-value chunk (16 bytes) to its K position 256 sb + ksub<SUB>() + coff(q).
// grid (ceil(row groups x columns / 4), n); P:11471-11498 contract, all four formats.
template <int TYPE, int SUB>
__device__ __forceinline__ void dequant_step(const uint8_t* row, int sb, int h, int64_t cols,
                                             const typename BPiece<TYPE>::Head& hd, const uint32_t* grid,
                                             uint16_t* orow) {
  using BP = BPiece<TYPE>;
  const int64_t k0 = 256 * (int64_t)sb + BP::template ksub<SUB>();
  // Q8_0 rows may end inside a super-block column (a piece is one 32-value block): the
  // pieces past the row's end are not loaded
  if (k0 + BP::off0(h) >= cols) return;
  typename BP::Raw raw;
  uint32_t v[16];
  BP::template load<SUB>(row, sb, h, grid, raw);
  BP::template decode<SUB>(hd, raw, grid, v);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int pos = (c < 2 ? BP::off0(h) : BP::off1(h)) + 8 * (c & 1);  // step position of chunk c
    const u32x4_t w = {v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
    *(u32x4_t*)(orow + k0 + BP::coff(pos / 8)) = w;
  }
}

template <int TYPE>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ raw, int64_t raw_stride,
                                                      int64_t rows, int64_t cols, int64_t rb,
                                                      uint16_t* __restrict__ out, int64_t out_stride) {
  using BP = BPiece<TYPE>;
  __shared__ uint32_t grid[TYPE == GGML_IQ3_S ? 512 : 1];
  if constexpr (TYPE == GGML_IQ3_S) {
    stage_iq3s_sel(grid);
    __syncthreads();
  }
  const int64_t e = blockIdx.y;
  const int lane = threadIdx.x & 63, h = lane >> 5;
  const int64_t nsb = (cols + 255) / 256;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (row group, column)
  if (unit >= (rows + 31) / 32 * nsb) return;
  const int64_t r = unit / nsb * 32 + (lane & 31);
  const int sb = (int)(unit % nsb);
  if (r >= rows) return;
  const uint8_t* row = raw + e * raw_stride + r * rb;
  uint16_t* orow = out + e * out_stride + r * cols;
  typename BP::Head hd;
  BP::load_head(row, sb, h, hd);
  dequant_step<TYPE, 0>(row, sb, h, cols, hd, grid, orow);
  dequant_step<TYPE, 1>(row, sb, h, cols, hd, grid, orow);
  dequant_step<TYPE, 2>(row, sb, h, cols, hd, grid, orow);
  dequant_step<TYPE, 3>(row, sb, h, cols, hd, grid, orow);
}

int launch_dequant(const uint8_t* raw, int64_t raw_stride, int type, int64_t n, int64_t rows, int64_t cols,
                   uint16_t* out, int64_t out_stride, hipStream_t stream) {
  const int64_t units = (rows + 31) / 32 * ((cols + 255) / 256);
  dim3 grid((unsigned)((units + 3) / 4), (unsigned)n);
  const int64_t rb = row_bytes(cols, type);
  switch (type) {
    case GGML_Q8_0: dequant_kernel<GGML_Q8_0><<<grid, 256, 0, stream>>>(raw, raw_stride, rows, cols, rb, out, out_stride); break;
    case GGML_Q4_K: dequant_kernel<GGML_Q4_K><<<grid, 256, 0, stream>>>(raw, raw_stride, rows, cols, rb, out, out_stride); break;
    case GGML_Q6_K: dequant_kernel<GGML_Q6_K><<<grid, 256, 0, stream>>>(raw, raw_stride, rows, cols, rb, out, out_stride); break;
    case GGML_IQ3_S: dequant_kernel<GGML_IQ3_S><<<grid, 256, 0, stream>>>(raw, raw_stride, rows, cols, rb, out, out_stride); break;
    default: set_error("dequant: ggml type %d has no kernel", type); return KTMI_ETYPE;
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

// ---------------------------------------------------------------- hot-cache route
// hot/kt_hot_cache.py:62-75: two table lookups and a count per route. fp32 counts of
// +1.0 stay exact below 2^24, so the atomic order does not change them.
__global__ __launch_bounds__(256) void route_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                    const int32_t* __restrict__ log2slot,
                                                    const int32_t* __restrict__ log2cpu, float* counts,
                                                    int32_t* __restrict__ slot_ids, int32_t* __restrict__ cpu_ids) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t e = ids[i];
  slot_ids[i] = log2slot[e];
  cpu_ids[i] = log2cpu[e];
  if (counts) atomicAdd(counts + e, 1.0f);
}

int launch_route(const int32_t* ids, int64_t n, const int32_t* log2slot, const int32_t* log2cpu, float* counts,
                 int32_t* slot_ids, int32_t* cpu_ids, hipStream_t stream) {
  if (n == 0) return KTMI_OK;
  route_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(ids, n, log2slot, log2cpu, counts, slot_ids, cpu_ids);
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

// ---------------------------------------------------------------- q8_1 quantisation
// kt_gguf_moe_multi.cu:600-650: one thread per value of the padded row; the 32 values
// of a block are 32 consecutive lanes (half a wave64). amax and sum reduce over the
// half-wave in xor-butterfly order; lane 0 of the block writes (half d, half sum).
template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<_Float16>(_Float16 v) { return (float)v; }
template <>
__device__ __forceinline__ float to_f32<__bf16>(__bf16 v) { return (float)v; }

template <typename T>
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const T* __restrict__ x, uint8_t* __restrict__ y,
                                                            int64_t kx, int64_t kx_padded, int64_t tokens) {
  const int64_t ix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t iy = blockIdx.y;
  if (ix >= kx_padded || iy >= tokens) return;  // kx_padded is a multiple of 512: whole waves exit
  const float xi = ix < kx ? to_f32<T>(x[iy * kx + ix]) : 0.0f;
  float amax = fabsf(xi);
  float sum = xi;
#pragma unroll
  for (int mask = 16; mask > 0; mask >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, mask, 32));
    sum += __shfl_xor(sum, mask, 32);
  }
  const float d = amax / 127.0f;
  const int8_t q = amax == 0.0f ? 0 : (int8_t)roundf(xi / d);
  uint8_t* blk = y + iy * (kx_padded / 32 * QB8_1) + (ix / 32) * QB8_1;
  blk[4 + (ix % 32)] = (uint8_t)q;
  if ((ix % 32) == 0) {
    *(uint32_t*)blk = (uint32_t)float_to_half_bits(d) | ((uint32_t)float_to_half_bits(sum) << 16);
  }
}

int launch_quantize_q8_1(const void* x, int dtype, int64_t cols, int64_t tokens, uint8_t* out, hipStream_t stream) {
  if (tokens == 0) return KTMI_OK;
  const int64_t kp = q8_1_cols_padded(cols);
  // grid.y is limited to 65535: slice the tokens
  for (int64_t t0 = 0; t0 < tokens; t0 += 65535) {
    const int64_t nt = tokens - t0 < 65535 ? tokens - t0 : 65535;
    dim3 grid((unsigned)(kp / 256), (unsigned)nt);
    uint8_t* o = out + t0 * (kp / 32 * QB8_1);
    switch (dtype) {
      case KTMI_F32: quantize_q8_1_kernel<float><<<grid, 256, 0, stream>>>((const float*)x + t0 * cols, o, cols, kp, nt); break;
      case KTMI_F16: quantize_q8_1_kernel<_Float16><<<grid, 256, 0, stream>>>((const _Float16*)x + t0 * cols, o, cols, kp, nt); break;
      case KTMI_BF16: quantize_q8_1_kernel<__bf16><<<grid, 256, 0, stream>>>((const __bf16*)x + t0 * cols, o, cols, kp, nt); break;
      default: set_error("quantize_q8_1: dtype %d", dtype); return KTMI_EINVAL;
    }
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

// ---------------------------------------------------------------- SiLU * mul
template <typename T>
__device__ __forceinline__ T from_f32(float v) { return (T)v; }

template <typename T>
__global__ __launch_bounds__(256) void silu_and_mul_kernel(const T* __restrict__ h, int64_t R, int64_t N,
                                                           T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= R * N) return;
  const int64_t r = i / N, n = i % N;
  const float g = to_f32<T>(h[r * 2 * N + n]);
  const float u = to_f32<T>(h[r * 2 * N + N + n]);
  out[i] = from_f32<T>(g / (1.0f + expf(-g)) * u);
}

int launch_silu_and_mul(const void* h, int dtype, int64_t R, int64_t N, void* out, hipStream_t stream) {
  const int64_t n = R * N;
  if (n == 0) return KTMI_OK;
  const unsigned g = (unsigned)((n + 255) / 256);
  switch (dtype) {
    case KTMI_F32: silu_and_mul_kernel<float><<<g, 256, 0, stream>>>((const float*)h, R, N, (float*)out); break;
    case KTMI_F16: silu_and_mul_kernel<_Float16><<<g, 256, 0, stream>>>((const _Float16*)h, R, N, (_Float16*)out); break;
    case KTMI_BF16: silu_and_mul_kernel<__bf16><<<g, 256, 0, stream>>>((const __bf16*)h, R, N, (__bf16*)out); break;
    default: set_error("silu_and_mul: dtype %d", dtype); return KTMI_EINVAL;
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

// ---------------------------------------------------------------- combine
// hot/kt_gguf_hot.py:43-71: res[t, c] = round(sum_k fp32(round(out[t,k,c] * round(w[t,k])))),
// k ascending, one thread per 4 columns of a token.
template <typename T>
__global__ __launch_bounds__(256) void combine_kernel(const T* __restrict__ out, const float* __restrict__ w,
                                                      int64_t T_, int top_k, int64_t K, T* __restrict__ res) {
  const int64_t t = blockIdx.y;
  const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= K) return;
  float acc = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    const float wk = to_f32<T>(from_f32<T>(w[t * top_k + k]));
    const float o = to_f32<T>(out[(t * top_k + k) * K + c]);
    acc += to_f32<T>(from_f32<T>(o * wk));
  }
  res[t * K + c] = from_f32<T>(acc);
}

int launch_combine(const void* out, int dtype, const float* w, int64_t T_, int64_t top_k, int64_t K, void* res,
                   hipStream_t stream) {
  if (T_ == 0 || K == 0) return KTMI_OK;
  for (int64_t t0 = 0; t0 < T_; t0 += 65535) {
    const int64_t nt = T_ - t0 < 65535 ? T_ - t0 : 65535;
    dim3 grid((unsigned)((K + 255) / 256), (unsigned)nt);
    switch (dtype) {
      case KTMI_F32:
        combine_kernel<float><<<grid, 256, 0, stream>>>((const float*)out + t0 * top_k * K, w + t0 * top_k, nt,
                                                        (int)top_k, K, (float*)res + t0 * K);
        break;
      case KTMI_F16:
        combine_kernel<_Float16><<<grid, 256, 0, stream>>>((const _Float16*)out + t0 * top_k * K, w + t0 * top_k, nt,
                                                           (int)top_k, K, (_Float16*)res + t0 * K);
        break;
      case KTMI_BF16:
        combine_kernel<__bf16><<<grid, 256, 0, stream>>>((const __bf16*)out + t0 * top_k * K, w + t0 * top_k, nt,
                                                         (int)top_k, K, (__bf16*)res + t0 * K);
        break;
      default: set_error("combine: dtype %d", dtype); return KTMI_EINVAL;
    }
  }
  KTMI_HIP_TRY(hipGetLastError());
  return KTMI_OK;
}

}  // namespace ktmi
