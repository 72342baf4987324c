// Greedy sampling: out[r] = argmax(logits[r, :]) over a (rows, vocab) matrix.
//
// Replaces _argmax_chunks_kernel + _argmax_rows_kernel
// (babyvllm/kernels/argmax.py:14-56). HBM-bound: 64 x 152,064 bf16 logits are
// 19.5 MB per decode step. Stage 1: work-group (row, chunk of kChunk columns),
// 256 threads reading 16 bytes per load, keeps each thread's best (value,
// index), reduces them in the wave and across the 4 waves, and writes the
// chunk's winner. Stage 2: one wave per row reduces the row's chunk winners.
//
// Order is torch.argmax's: the larger value wins, equal values go to the lower
// index, and NaN counts as larger than any number (the first NaN wins).
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

namespace {

constexpr int kArgmaxThreads = 256;
constexpr int kChunk = 4096;  // columns per stage-1 work-group

struct Best {
  float v;
  int i;
};

// True if (v, i) comes before (w, j) in argmax order.
__device__ __forceinline__ bool better(float v, int i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  if (vn || wn) return vn && (!wn || i < j);
  return v > w || (v == w && i < j);
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float w = __shfl_xor(b.v, off, 64);
    const int j = __shfl_xor(b.i, off, 64);
    if (better(w, j, b.v, b.i)) {
      b.v = w;
      b.i = j;
    }
  }
  return b;
}

// Work-group best of 4 waves' bests, in wave order through LDS.
__device__ __forceinline__ Best block_best(Best b) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  b = wave_best(b);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = b.v;
    si[w] = b.i;
  }
  __syncthreads();
  Best r{sv[0], si[0]};
#pragma unroll
  for (int k = 1; k < kArgmaxThreads / 64; ++k)
    if (better(sv[k], si[k], r.v, r.i)) r = Best{sv[k], si[k]};
  return r;
}

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) { return bf16_to_f32(x); }
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }

// T = uint16_t (bf16 bits) or float. VEC elements per 16-byte load.
template <typename T, bool ALIGNED>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_chunks_kernel(const T* __restrict__ logits,
                                                                      int64_t row_stride, int vocab,
                                                                      int n_chunks, float* part_v,
                                                                      int* part_i) {
  constexpr int VEC = 16 / sizeof(T);
  const int row = blockIdx.x / n_chunks;
  const int chunk = blockIdx.x - row * n_chunks;
  const T* x = logits + (int64_t)row * row_stride;
  const int lo = chunk * kChunk;
  const int hi = min(lo + kChunk, vocab);
  Best b{-__builtin_huge_valf(), 0x7fffffff};
  if (ALIGNED) {
    // All of a thread's 16-byte vectors are requested before the first is
    // used. The thread's maximum is taken with plain max operations (and a
    // NaN flag), then its first column holding that maximum (or its first
    // NaN) is found: fewer operations per element than a running comparison.
    constexpr int PER = kChunk / (kArgmaxThreads * VEC);
    uint4 raw[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int c = lo + (threadIdx.x + k * kArgmaxThreads) * VEC;
      raw[k] = c < hi ? ld16(x + c) : make_uint4(0, 0, 0, 0);
    }
    // Max and NaN flag as trees over the thread's PER·VEC elements (short
    // dependence chains), then the first column holding the max (or the first
    // NaN) as a tree of minima over candidate columns.
    constexpr int NE = PER * VEC;
    float vals[NE];
    int cols[NE];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int c = lo + (threadIdx.x + k * kArgmaxThreads) * VEC;
      const T* e = reinterpret_cast<const T*>(&raw[k]);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        cols[k * VEC + j] = c + j;
        vals[k * VEC + j] = c + j < hi ? to_f32<T>(e[j]) : -__builtin_huge_valf();
      }
    }
    float mx[NE];
    bool nn[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) { mx[i] = vals[i]; nn[i] = vals[i] != vals[i]; }
#pragma unroll
    for (int s = 1; s < NE; s *= 2)
#pragma unroll
      for (int i = 0; i + s < NE; i += 2 * s) { mx[i] = fmaxf(mx[i], mx[i + s]); nn[i] = nn[i] || nn[i + s]; }
    const float m = mx[0];
    const bool any_nan = nn[0];
    int fi[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const float v = vals[i];
      const bool hit = cols[i] < hi && (any_nan ? v != v : v == m);
      fi[i] = hit ? cols[i] : 0x7fffffff;
    }
#pragma unroll
    for (int s = 1; s < NE; s *= 2)
#pragma unroll
      for (int i = 0; i + s < NE; i += 2 * s) fi[i] = min(fi[i], fi[i + s]);
    const int first = fi[0];
    if (first != 0x7fffffff) {
      b.v = any_nan ? __builtin_nanf("") : m;
      b.i = first;
    }
  } else {
    for (int c = lo + threadIdx.x; c < hi; c += kArgmaxThreads) {
      const float v = to_f32<T>(x[c]);
      if (better(v, c, b.v, b.i)) {
        b.v = v;
        b.i = c;
      }
    }
  }
  b = block_best(b);
  if (threadIdx.x == 0) {
    part_v[blockIdx.x] = b.v;
    part_i[blockIdx.x] = b.i;
  }
}

__global__ __launch_bounds__(64) void argmax_rows_kernel(const float* part_v, const int* part_i, int n_chunks,
                                                         int64_t* out) {
  const int row = blockIdx.x;
  Best b{-__builtin_huge_valf(), 0x7fffffff};
  for (int k = threadIdx.x; k < n_chunks; k += 64) {
    const float v = part_v[row * n_chunks + k];
    const int i = part_i[row * n_chunks + k];
    if (better(v, i, b.v, b.i)) {
      b.v = v;
      b.i = i;
    }
  }
  b = wave_best(b);
  if (threadIdx.x == 0) out[row] = b.i;
}

template <typename T>
hipError_t launch_argmax(const ArgmaxArgs& a, hipStream_t stream) {
  const int n_chunks = (a.vocab + kChunk - 1) / kChunk;
  const int64_t wgs = (int64_t)a.rows * n_chunks;
  if (wgs > 0x7fffffff) return hipErrorInvalidValue;
  const T* x = reinterpret_cast<const T*>(a.logits);
  float* pv = reinterpret_cast<float*>(a.workspace);
  int* pi = reinterpret_cast<int*>(pv + wgs);
  if (a.vec_ok)
    hipLaunchKernelGGL((argmax_chunks_kernel<T, true>), dim3((unsigned)wgs), dim3(kArgmaxThreads), 0, stream, x,
                       a.row_stride, a.vocab, n_chunks, pv, pi);
  else
    hipLaunchKernelGGL((argmax_chunks_kernel<T, false>), dim3((unsigned)wgs), dim3(kArgmaxThreads), 0, stream, x,
                       a.row_stride, a.vocab, n_chunks, pv, pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)a.rows), dim3(64), 0, stream, pv, pi, n_chunks, a.out);
  return hipGetLastError();
}

}  // namespace

int64_t argmax_workspace_bytes(int32_t rows, int32_t vocab) {
  const int64_t n_chunks = ((int64_t)vocab + kChunk - 1) / kChunk;
  return (int64_t)rows * n_chunks * 8;
}

hipError_t greedy_argmax(const ArgmaxArgs& a, hipStream_t stream) {
  return a.fp32 ? launch_argmax<float>(a, stream) : launch_argmax<uint16_t>(a, stream);
}

}  // namespace bvllm
