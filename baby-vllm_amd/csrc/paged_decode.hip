// Paged decode attention: one query token per sequence against its paged K/V,
// with the flash-decoding split (partial softmax per split + LSE reduce).
//
// Replaces paged_decode_attn_kernel, paged_decode_attn_split_kernel and
// paged_decode_attn_reduce_kernel (babyvllm/kernels/paged_attn.py:9-251).
// The work-group body (page walk, MFMA products, in-LDS merge of the waves) is
// decode_work_group in paged_decode_wg.h; this file holds the kernels that
// launch it, the split reduce, and the launch choices.
#include "paged_decode_wg.h"

#include <stdlib.h>

#include <algorithm>

namespace bvllm {

template <int D, int NW, int PF>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_work_group<D, NW, PF>(a, blockIdx.x, smem);
}

// One work-group per (sequence, query head, 32-dim slice):
//   out = Σ_s w_s·o_s / Σ_s w_s,  w_s = 2^(lse_s − max lse).
// Thread (chunk, group) accumulates splits group, group + 32, ... in order, then
// the 32 group sums are added in group order. The grouping depends only on the
// split index, so trailing empty splits (w = 0, o = 0) leave the bits unchanged.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeArgs a) {
  constexpr int DS = 32;          // dims per work-group
  constexpr int CH = DS / 4;      // float4 chunks per slice
  constexpr int NG = 256 / CH;    // split groups
  constexpr int SLICES = D / DS;
  __shared__ float red[256];
  __shared__ float4 gnum[NG][CH];
  __shared__ float gden[NG];

  const int bh = blockIdx.x / SLICES;
  const int d0 = (blockIdx.x % SLICES) * DS;
  const int S = a.num_splits;
  const float* lse = a.part_lse + (int64_t)bh * S;
  const float* po = a.part_out + (int64_t)bh * S * D + d0;

  float M = kNegInf;
  for (int s = threadIdx.x; s < S; s += 256) M = fmaxf(M, lse[s]);
  red[threadIdx.x] = M;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + off]);
    __syncthreads();
  }
  M = red[0];
  if (M == kNegInf) M = 0.f;

  const int ch = threadIdx.x % CH;
  const int grp = threadIdx.x / CH;
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f;
#pragma unroll 4
  for (int s = grp; s < S; s += NG) {
    const float wgt = fast_exp2(lse[s] - M);
    const float4 x = *reinterpret_cast<const float4*>(po + (int64_t)s * D + 4 * ch);
    num.x += wgt * x.x;
    num.y += wgt * x.y;
    num.z += wgt * x.z;
    num.w += wgt * x.w;
    den += wgt;
  }
  gnum[grp][ch] = num;
  if (ch == 0) gden[grp] = den;
  __syncthreads();
  if (grp == 0) {
    float4 t = gnum[0][ch];
    float dd = gden[0];
    for (int q = 1; q < NG; ++q) {
      const float4 x = gnum[q][ch];
      t.x += x.x;
      t.y += x.y;
      t.z += x.z;
      t.w += x.w;
      dd += gden[q];
    }
    const float inv = 1.f / (dd == 0.f ? 1.f : dd);
    const int b = bh / a.num_heads;
    const int h = bh % a.num_heads;
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d0 + 4 * ch;
    uint2 pk;
    pk.x = pack_bf16x2_hw(t.x * inv, t.y * inv);
    pk.y = pack_bf16x2_hw(t.z * inv, t.w * inv);
    st8(dst, pk);
  }
}

// Reduce for at most 32 partial states per (row, head): one thread per
// (row, head, 4 dims) accumulates the partials in order. With ≤ 32 partials
// every group of decode_reduce_kernel holds at most one non-empty partial, so
// both kernels return the same bits for the same row (trailing empty partials
// add exact zeros in either).
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_small_kernel(DecodeArgs a, int64_t items) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= items) return;
  const int64_t bh = t / (D / 4);
  const int d = (int)(t - bh * (D / 4)) * 4;
  const int S = a.num_splits;
  const float* lse = a.part_lse + bh * S;
  const float* po = a.part_out + bh * S * D + d;
  float M = kNegInf;
#pragma unroll 8
  for (int s = 0; s < S; ++s) M = fmaxf(M, lse[s]);
  if (M == kNegInf) M = 0.f;
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f;
#pragma unroll 8
  for (int s = 0; s < S; ++s) {
    const float wgt = fast_exp2(lse[s] - M);
    const float4 x = *reinterpret_cast<const float4*>(po + (int64_t)s * D);
    num.x += wgt * x.x;
    num.y += wgt * x.y;
    num.z += wgt * x.z;
    num.w += wgt * x.w;
    den += wgt;
  }
  const float inv = 1.f / (den == 0.f ? 1.f : den);
  const int b = (int)(bh / a.num_heads);
  const int h = (int)(bh % a.num_heads);
  uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d;
  uint2 pk;
  pk.x = pack_bf16x2_hw(num.x * inv, num.y * inv);
  pk.y = pack_bf16x2_hw(num.z * inv, num.w * inv);
  st8(dst, pk);
}

template <int D>
static hipError_t launch_reduce(const DecodeArgs& r, hipStream_t stream) {
  if (r.num_splits <= 32) {
    const int64_t items = (int64_t)r.batch * r.num_heads * (D / 4);
    hipLaunchKernelGGL((decode_reduce_small_kernel<D>), dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       stream, r, items);
  } else {
    hipLaunchKernelGGL((decode_reduce_kernel<D>), dim3((unsigned)(r.batch * r.num_heads * (D / 32))), dim3(256),
                       0, stream, r);
  }
  return hipGetLastError();
}

template <int D, int NW, int PF>
static hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const int G = a.num_heads / a.num_kv_heads;
  const size_t smem = decode_lds_bytes<D, NW>(G);
  if (smem > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_decode_kernel<D, NW, PF>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int64_t wgs = (int64_t)a.batch * a.num_kv_heads * a.num_splits;
  if (wgs == 0) return hipSuccess;
  if (wgs > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_decode_kernel<D, NW, PF>), dim3((unsigned)wgs), dim3(NW * 64), smem, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || a.num_splits == 1) return err;
  return launch_reduce<D>(a, stream);
}

// Pages in flight per wave; BVLLM_DECODE_DEPTH (2, 3 or 4) overrides the default for tuning.
// Two is best measured on MI355X: deeper queues lose DRAM efficiency on the
// 256-byte head slices.
static int decode_depth() {
  static const int depth = [] {
    const char* e = getenv("BVLLM_DECODE_DEPTH");
    const int v = e ? atoi(e) : 0;
    return (v >= 2 && v <= 4) ? v : 2;
  }();
  return depth;
}

template <int D, int NW>
static hipError_t decode_for_depth(const DecodeArgs& a, hipStream_t stream) {
  switch (decode_depth()) {
    case 2: return launch_decode<D, NW, 2>(a, stream);
    case 4: return launch_decode<D, NW, 4>(a, stream);
    default: return launch_decode<D, NW, 3>(a, stream);
  }
}

template <int D>
static hipError_t decode_for_dim(const DecodeArgs& a, hipStream_t stream) {
  switch (a.waves) {
    case 4: return decode_for_depth<D, 4>(a, stream);
    case 8: return decode_for_depth<D, 8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

int32_t decode_partials(const DecodeArgs& a) { return a.num_splits; }

hipError_t paged_decode(const DecodeArgs& a, hipStream_t stream) {
  DecodeArgs d = a;
  if (d.waves == 0) d.waves = 4;
  switch (a.head_dim) {
    case 64: return decode_for_dim<64>(d, stream);
    case 128: return decode_for_dim<128>(d, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
