// Greedy sampling: out[r] = argmax(logits[r, :]) over a (rows, vocab) matrix.
//
// Replaces _argmax_chunks_kernel + _argmax_rows_kernel
// (babyvllm/kernels/argmax.py:14-56). HBM-bound: 64 x 152,064 bf16 logits are
// 19.5 MB per decode step. Stage 1: work-group = (chunk of columns, row), 256
// threads; it writes the chunk's maximum and the first column holding it.
// Stage 2: one wave per row merges the row's chunk results.
//
// Order is torch.argmax's: the larger value wins, equal values go to the lower
// index (-0.0 equals +0.0), and NaN counts as larger than any number (the first
// NaN wins).
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

namespace {

constexpr int kArgmaxThreads = 256;
constexpr int kVecLoads = 2;        // 16-byte loads per thread on aligned rows
constexpr int kScalarChunk = 4096;  // columns per work-group on unaligned rows
constexpr int kMaxGridY = 65535;    // rows per launch (grid y)

template <typename T>
constexpr int vec_chunk() { return kVecLoads * kArgmaxThreads * (16 / (int)sizeof(T)); }

// ------------------------------------------------------ wave reductions
//
// Wave-wide maximum / minimum by DPP and lane swaps (VALU only, no LDS round
// trip): quad swaps (lanes l ^ 1, then l ^ 2), mirrors within 8 and within 16
// lanes, then the 16- and 32-lane swaps. Each step combines a lane with a
// partner holding the other half of its current group, so every lane ends
// with the result for the whole wave.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, 0xf, 0xf, false);
}
constexpr int kQuadSwap1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int kQuadSwap2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// NaN-propagating: the result is NaN if any lane holds a NaN.
__device__ __forceinline__ float wave_maximum(float x) {
  x = fmax_prop(x, __uint_as_float(dpp<kQuadSwap1>(__float_as_uint(x))));
  x = fmax_prop(x, __uint_as_float(dpp<kQuadSwap2>(__float_as_uint(x))));
  x = fmax_prop(x, __uint_as_float(dpp<kRowHalfMirror>(__float_as_uint(x))));
  x = fmax_prop(x, __uint_as_float(dpp<kRowMirror>(__float_as_uint(x))));
  return max_across_groups(x);
}

__device__ __forceinline__ int wave_min(int x) {
  x = min(x, (int)dpp<kQuadSwap1>((uint32_t)x));
  x = min(x, (int)dpp<kQuadSwap2>((uint32_t)x));
  x = min(x, (int)dpp<kRowHalfMirror>((uint32_t)x));
  x = min(x, (int)dpp<kRowMirror>((uint32_t)x));
  const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
  x = min((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
  return min((int)b[0], (int)b[1]);
}

// Work-group maximum (NaN-propagating) and minimum over the 4 waves, through
// LDS; every thread gets the result. `slot` is 4 floats / ints of LDS.
__device__ __forceinline__ float group_maximum(float x, float* slot) {
  x = wave_maximum(x);
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmax_prop(fmax_prop(slot[0], slot[1]), fmax_prop(slot[2], slot[3]));
}
__device__ __forceinline__ int group_min(int x, int* slot) {
  x = wave_min(x);
  if ((threadIdx.x & 63) == 0) slot[threadIdx.x >> 6] = x;
  __syncthreads();
  return min(min(slot[0], slot[1]), min(slot[2], slot[3]));
}
static_assert(kArgmaxThreads == 4 * 64, "group reductions combine four waves");

// ------------------------------------------------------------- stage 1

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) { return bf16_to_f32(x); }
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }

// Element j of a 16-byte vector of T, as fp32.
template <typename T>
__device__ __forceinline__ float vec_elem(const uint4& r, int j);
template <>
__device__ __forceinline__ float vec_elem<uint16_t>(const uint4& r, int j) {
  const uint32_t w = (&r.x)[j >> 1];
  return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float vec_elem<float>(const uint4& r, int j) { return __uint_as_float((&r.x)[j]); }

// A 16-byte vector of -inf (stands for the columns past the row's end).
template <typename T>
__device__ __forceinline__ uint4 neg_inf_vec();
template <>
__device__ __forceinline__ uint4 neg_inf_vec<uint16_t>() { return make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u); }
template <>
__device__ __forceinline__ uint4 neg_inf_vec<float>() { return make_uint4(0xff800000u, 0xff800000u, 0xff800000u, 0xff800000u); }

// Aligned rows (16-byte loads cover whole rows): thread t reads the 16-byte
// vectors t and t + 256 of the chunk, both requested before either is used,
// with the nontemporal hint (the logits are read once). The work-group's
// maximum is formed first (NaN-propagating max trees, then DPP and LDS); then
// only the threads holding it look for its first column among their elements
// (a NaN maximum: the first NaN), and the smallest such column wins. Vectors
// past the row's end read as -inf and lie at higher columns than every real
// one, so they never win: a chunk holds at least one real column.
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_chunks_vec_kernel(const T* __restrict__ logits,
                                                                          int64_t row_stride, int vocab,
                                                                          int n_chunks, float* part_v,
                                                                          int* part_i) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int NE = kVecLoads * VEC;
  constexpr int CHUNK = vec_chunk<T>();
  __shared__ float smax[4];
  __shared__ int smin[4];
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const T* x = logits + (int64_t)row * row_stride;
  const int lo = chunk * CHUNK;
  const int c0 = lo + (int)threadIdx.x * VEC;
  uint4 raw[kVecLoads];
  if (lo + CHUNK <= vocab) {
#pragma unroll
    for (int k = 0; k < kVecLoads; ++k) raw[k] = ld16_nt(x + c0 + k * kArgmaxThreads * VEC);
  } else {
#pragma unroll
    for (int k = 0; k < kVecLoads; ++k) {
      const int c = c0 + k * kArgmaxThreads * VEC;
      raw[k] = c < vocab ? ld16_nt(x + c) : neg_inf_vec<T>();
    }
  }
  float v[NE];
#pragma unroll
  for (int k = 0; k < kVecLoads; ++k)
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[k * VEC + j] = vec_elem<T>(raw[k], j);
  float mx[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) mx[e] = v[e];
#pragma unroll
  for (int s = 1; s < NE; s *= 2)
#pragma unroll
    for (int e = 0; e + s < NE; e += 2 * s) mx[e] = fmax_prop(mx[e], mx[e + s]);
  const float mt = mx[0];
  // Uniform across the work-group, so each search below is one branch.
  const float M = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(group_maximum(mt, smax))));
  int col = 0x7fffffff;
  if (M == M) {
    if (mt == M) {
      int first = 0;
#pragma unroll
      for (int e = NE - 1; e >= 0; --e) first = v[e] == M ? e : first;
      col = c0 + (first / VEC) * kArgmaxThreads * VEC + first % VEC;
    }
  } else if (mt != mt) {
    int first = 0;
#pragma unroll
    for (int e = NE - 1; e >= 0; --e) first = v[e] != v[e] ? e : first;
    col = c0 + (first / VEC) * kArgmaxThreads * VEC + first % VEC;
  }
  col = group_min(col, smin);
  if (threadIdx.x == 0) {
    part_v[(int64_t)row * n_chunks + chunk] = M;
    part_i[(int64_t)row * n_chunks + chunk] = col;
  }
}

// True if (v, i) comes before (w, j) in argmax order.
__device__ __forceinline__ bool better(float v, int i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  if (vn || wn) return vn && (!wn || i < j);
  return v > w || (v == w && i < j);
}

// Unaligned rows (a view whose rows are not 16-byte vectors): element loads,
// each thread keeps its best (value, column) by running comparison, then the
// work-group's best (the same order as above: maximum first, then the
// smallest column holding it).
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_chunks_scalar_kernel(const T* __restrict__ logits,
                                                                             int64_t row_stride, int vocab,
                                                                             int n_chunks, float* part_v,
                                                                             int* part_i) {
  __shared__ float smax[4];
  __shared__ int smin[4];
  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const T* x = logits + (int64_t)row * row_stride;
  const int lo = chunk * kScalarChunk;
  const int hi = min(lo + kScalarChunk, vocab);
  float bv = -__builtin_huge_valf();
  int bi = 0x7fffffff;
  for (int c = lo + (int)threadIdx.x; c < hi; c += kArgmaxThreads) {
    const float v = to_f32<T>(x[c]);
    if (better(v, c, bv, bi)) {
      bv = v;
      bi = c;
    }
  }
  const float M = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(group_maximum(bv, smax))));
  const int col = group_min((M == M ? bv == M : bv != bv) ? bi : 0x7fffffff, smin);
  if (threadIdx.x == 0) {
    part_v[(int64_t)row * n_chunks + chunk] = M;
    part_i[(int64_t)row * n_chunks + chunk] = col;
  }
}

// ------------------------------------------------------------- stage 2

// One wave per row: the largest chunk maximum (NaN if any chunk's is), then
// the smallest column among the chunks holding it.
__global__ __launch_bounds__(64) void argmax_rows_kernel(const float* part_v, const int* part_i, int n_chunks,
                                                         int64_t* out) {
  const int row = blockIdx.x;
  const float* pv = part_v + (int64_t)row * n_chunks;
  const int* pi = part_i + (int64_t)row * n_chunks;
  float m = -__builtin_huge_valf();
  for (int k = threadIdx.x; k < n_chunks; k += 64) m = fmax_prop(m, pv[k]);
  const float M = wave_maximum(m);
  int col = 0x7fffffff;
  for (int k = threadIdx.x; k < n_chunks; k += 64) {
    const float v = pv[k];
    if (M == M ? v == M : v != v) col = min(col, pi[k]);
  }
  col = wave_min(col);
  if (threadIdx.x == 0) out[row] = col;
}

template <typename T>
hipError_t launch_argmax(const ArgmaxArgs& a, hipStream_t stream) {
  const int chunk = a.vec_ok ? vec_chunk<T>() : kScalarChunk;
  const int n_chunks = (a.vocab + chunk - 1) / chunk;
  float* pv = reinterpret_cast<float*>(a.workspace);
  int* pi = reinterpret_cast<int*>(pv + (int64_t)a.rows * n_chunks);
  const T* x = reinterpret_cast<const T*>(a.logits);
  for (int r0 = 0; r0 < a.rows; r0 += kMaxGridY) {
    const int rows = min(kMaxGridY, a.rows - r0);
    const T* xr = x + (int64_t)r0 * a.row_stride;
    float* pvr = pv + (int64_t)r0 * n_chunks;
    int* pir = pi + (int64_t)r0 * n_chunks;
    const dim3 grid((unsigned)n_chunks, (unsigned)rows);
    if (a.vec_ok)
      hipLaunchKernelGGL(argmax_chunks_vec_kernel<T>, grid, dim3(kArgmaxThreads), 0, stream, xr, a.row_stride,
                         a.vocab, n_chunks, pvr, pir);
    else
      hipLaunchKernelGGL(argmax_chunks_scalar_kernel<T>, grid, dim3(kArgmaxThreads), 0, stream, xr, a.row_stride,
                         a.vocab, n_chunks, pvr, pir);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(64), 0, stream, pvr, pir, n_chunks, a.out + r0);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

// Sized for the most chunks any path uses (fp32 aligned rows: vec_chunk<float>()
// columns per chunk): one (value, column) pair of 8 bytes per chunk.
int64_t argmax_workspace_bytes(int32_t rows, int32_t vocab) {
  constexpr int kSmallestChunk = vec_chunk<float>();
  static_assert(kSmallestChunk <= vec_chunk<uint16_t>() && kSmallestChunk <= kScalarChunk, "smallest chunk");
  const int64_t n_chunks = ((int64_t)vocab + kSmallestChunk - 1) / kSmallestChunk;
  return (int64_t)rows * n_chunks * 8;
}

hipError_t greedy_argmax(const ArgmaxArgs& a, hipStream_t stream) {
  return a.fp32 ? launch_argmax<float>(a, stream) : launch_argmax<uint16_t>(a, stream);
}

}  // namespace bvllm
