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
#include <atomic>

namespace bvllm {

template <int D, int NW, int PF>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_work_group<D, NW, PF>(a, blockIdx.x, smem);
}

// Many short splits: one split per wave (decode_split_wave), one wave per
// work-group, so that a short batch's splits spread over every CU (B8 x 1920:
// 480 splits on 480 work-groups instead of 120 four-wave ones, 15.5 -> 14.1 us;
// two waves per work-group 14.4, four pages in flight per wave slower at any
// work-group size).
template <int D, int PF>
__global__ __launch_bounds__(64) void paged_decode_split_wave_kernel(DecodeArgs a, int items) {
  __shared__ __attribute__((aligned(16))) unsigned char tile[kTileBytes<D>];
  const int item = (int)blockIdx.x;
  if (item >= items) return;
  decode_split_wave<D, PF>(a, item, tile);
}

// Split reduce: out = Σ_s w_s·o_s / Σ_s w_s, w_s = 2^(lse_s − max lse), over the
// S partial states of a (row, head). Both reduce kernels use the same
// arithmetic, so a row's bits do not depend on S beyond its empty splits
// (w = 0, o = 0; eager and graph launches differ only in those):
//   * splits are taken in groups of kReduceGroup consecutive splits; a group's
//     sums are fma chains in split order: num = fma(w_s, o_s, num), den += w_s;
//   * group sums are added in group order, skipping groups with den == 0.
// With S ≤ kReduceGroup there is one group and its chain is the result.
constexpr int kReduceGroup = 32;

// One group's partial states for 4 dims, loaded in one round.
struct ReduceGroup {
  float l[kReduceGroup];
  float4 x[kReduceGroup];
};

__device__ __forceinline__ void load_group(ReduceGroup& r, const float* lse, const float* po, int D, int s0,
                                           int S) {
#pragma unroll
  for (int k = 0; k < kReduceGroup; ++k) {
    const int s = s0 + k;
    r.l[k] = s < S ? lse[s] : kNegInf;
    r.x[k] = s < S ? *reinterpret_cast<const float4*>(po + (int64_t)s * D) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

__device__ __forceinline__ float group_max(const ReduceGroup& r) {
  float M = kNegInf;
#pragma unroll
  for (int k = 0; k < kReduceGroup; ++k) M = fmaxf(M, r.l[k]);
  return M;
}

// The group's fma chains in split order.
__device__ __forceinline__ void chain_group(const ReduceGroup& r, float M, float4& num, float& den) {
  num = make_float4(0.f, 0.f, 0.f, 0.f);
  den = 0.f;
#pragma unroll
  for (int k = 0; k < kReduceGroup; ++k) {
    const float wgt = fast_exp2(r.l[k] - M);
    num.x = __builtin_fmaf(wgt, r.x[k].x, num.x);
    num.y = __builtin_fmaf(wgt, r.x[k].y, num.y);
    num.z = __builtin_fmaf(wgt, r.x[k].z, num.z);
    num.w = __builtin_fmaf(wgt, r.x[k].w, num.w);
    den += wgt;
  }
}

__device__ __forceinline__ void store_reduced(const DecodeArgs& a, int64_t bh, int d, float4 num, float den) {
  const float inv = 1.f / (den == 0.f ? 1.f : den);
  const int b = (int)(bh / a.num_heads);
  const int h = (int)(bh % a.num_heads);
  uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d;
  uint2 pk;
  pk.x = pack_bf16x2_hw(num.x * inv, num.y * inv);
  pk.y = pack_bf16x2_hw(num.z * inv, num.w * inv);
  st8(dst, pk);
}

// S ≤ kReduceGroup: one thread per (row, head, 4 dims), one group.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_small_kernel(DecodeArgs a, int64_t items) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= items) return;
  const int64_t bh = t / (D / 4);
  const int d = (int)(t - bh * (D / 4)) * 4;
  const int S = a.num_splits;
  ReduceGroup r;
  load_group(r, a.part_lse + bh * S, a.part_out + bh * S * D + d, D, 0, S);
  float M = group_max(r);
  if (M == kNegInf) M = 0.f;
  float4 num;
  float den;
  chain_group(r, M, num, den);
  store_reduced(a, bh, d, num, den);
}

// S > kReduceGroup: one work-group per (row, head, 32-dim slice); thread
// (chunk, q) sums group q of the current set of 32 groups, then the threads of
// group 0 add the set's group sums in order onto the running total.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeArgs a) {
  constexpr int DS = 32;          // dims per work-group
  constexpr int CH = DS / 4;      // float4 chunks per slice
  constexpr int NQ = 256 / CH;    // groups per set
  constexpr int SLICES = D / DS;
  __shared__ float red[256];
  __shared__ float4 gnum[NQ][CH];
  static_assert(NQ <= 256, "max pass scratch");
  __shared__ float gden[NQ];

  const int64_t bh = blockIdx.x / SLICES;
  const int d0 = (blockIdx.x % SLICES) * DS;
  const int S = a.num_splits;
  const float* lse = a.part_lse + bh * S;
  const float* po = a.part_out + bh * S * D + d0;

  const int ch = threadIdx.x % CH;
  const int q = threadIdx.x / CH;
  ReduceGroup r;
  float M;
  if (S <= NQ * kReduceGroup) {
    // One set: the group loads double as the max pass.
    load_group(r, lse, po + 4 * ch, D, q * kReduceGroup, S);
    if (ch == 0) red[q] = group_max(r);
    __syncthreads();
    M = kNegInf;
    for (int k = 0; k < NQ; ++k) M = fmaxf(M, red[k]);
  } else {
    M = kNegInf;
    for (int s = threadIdx.x; s < S; s += 256) M = fmaxf(M, lse[s]);
    red[threadIdx.x] = M;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
      if ((int)threadIdx.x < off) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + off]);
      __syncthreads();
    }
    M = red[0];
  }
  if (M == kNegInf) M = 0.f;

  float4 total = make_float4(0.f, 0.f, 0.f, 0.f);
  float total_den = 0.f;
  bool any = false;
  for (int set0 = 0; set0 < S; set0 += NQ * kReduceGroup) {
    if (set0 > 0 || S > NQ * kReduceGroup) load_group(r, lse, po + 4 * ch, D, set0 + q * kReduceGroup, S);
    float4 num;
    float den;
    chain_group(r, M, num, den);
    gnum[q][ch] = num;
    if (ch == 0) gden[q] = den;
    __syncthreads();
    if (q == 0) {
      for (int k = 0; k < NQ; ++k) {
        if (gden[k] == 0.f) continue;
        const float4 g = gnum[k][ch];
        if (!any) {
          total = g;
          total_den = gden[k];
          any = true;
        } else {
          total.x += g.x;
          total.y += g.y;
          total.z += g.z;
          total.w += g.w;
          total_den += gden[k];
        }
      }
    }
    __syncthreads();
  }
  if (q == 0) store_reduced(a, bh, d0 + 4 * ch, total, total_den);
}

template <int D>
static hipError_t launch_reduce(const DecodeArgs& r, hipStream_t stream) {
  if (r.num_splits <= kReduceGroup) {
    const int64_t items = (int64_t)r.batch * r.num_heads * (D / 4);
    hipLaunchKernelGGL((decode_reduce_small_kernel<D>), dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       stream, r, items);
  } else {
    hipLaunchKernelGGL((decode_reduce_kernel<D>), dim3((unsigned)(r.batch * r.num_heads * (D / 32))), dim3(256),
                       0, stream, r);
  }
  return hipGetLastError();
}

// Compute units of the current device (cached per device; host threads that
// race on the first query store the same value).
int device_cus() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Consecutive splits per work-group: about two work-groups per compute unit
// when the plan has more (small splits of a short batch, e.g. 512 splits of 4
// pages at batch 1: 4 splits per work-group, 33.7 instead of 37.5 us on
// MI355X), so that each work-group streams several splits' pages back to back.
// BVLLM_DECODE_SPLITS_PER_WG overrides the choice for tuning.
static int decode_splits_per_wg(const DecodeArgs& a, int nw) {
  if (a.num_splits <= 1 || a.blocks_per_split % nw != 0) return 1;
  const char* env = getenv("BVLLM_DECODE_SPLITS_PER_WG");  // read per launch: tests vary it
  const int forced = env ? atoi(env) : 0;
  int64_t gps;
  if (forced > 0) {
    gps = forced;
  } else {
    const int64_t cus = device_cus();
    const int64_t total = (int64_t)a.batch * a.num_kv_heads * a.num_splits;
    gps = (total + cus) / (2 * cus);
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>(gps, a.num_splits));
}

// Splits of at most this many pages run one per wave (decode_split_wave):
// with 4 or 8 pages per split the work-group path spends most of a split in
// its cross-wave merge. BVLLM_DECODE_SPLIT_WAVES=0 / 1 forces the work-group
// / the per-wave path for any split plan (read per launch: tests vary it).
constexpr int kSplitWaveMaxPages = 8;
static bool use_split_waves(const DecodeArgs& a) {
  if (a.num_splits <= 1 || a.waves != 4 || a.query_start_loc != nullptr) return false;
  const char* env = getenv("BVLLM_DECODE_SPLIT_WAVES");
  if (env && env[0] == '0') return false;
  if (env && env[0] == '1') return true;
  return a.blocks_per_split <= kSplitWaveMaxPages;
}

template <int D>
static hipError_t launch_split_waves(const DecodeArgs& a, hipStream_t stream) {
  const int64_t items = (int64_t)a.batch * a.num_kv_heads * a.num_splits;
  if (items == 0) return hipSuccess;
  if (items > 0x7ffffff0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_decode_split_wave_kernel<D, 2>), dim3((unsigned)items), dim3(64), 0, stream, a,
                     (int)items);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  return launch_reduce<D>(a, stream);
}

template <int D, int NW, int PF>
static hipError_t launch_decode(const DecodeArgs& args, hipStream_t stream) {
  DecodeArgs a = args;
  if (use_split_waves(a)) return launch_split_waves<D>(a, stream);
  a.splits_per_wg = decode_splits_per_wg(a, NW);
  const int G = a.num_heads / a.num_kv_heads;
  const size_t smem = decode_lds_bytes<D, NW>(G);
  if (smem > 160 * 1024) return hipErrorInvalidValue;
  // The dynamic-LDS limit is a per-device function attribute: set once per
  // device (setting it twice, from racing host threads, is harmless).
  static std::atomic<bool> attr_set[64] = {};
  int dev = 0;
  hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess) return de;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&paged_decode_kernel<D, NW, PF>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set[dev].store(true, std::memory_order_release);
  }
  const int64_t groups = (a.num_splits + a.splits_per_wg - 1) / a.splits_per_wg;
  const int64_t wgs = (int64_t)a.batch * a.num_kv_heads * groups;
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
