// Paged decode attention: one query token per sequence against its paged K/V,
// with the flash-decoding split (partial softmax per split + LSE reduce).
//
// Replaces paged_decode_attn_kernel, paged_decode_attn_split_kernel and
// paged_decode_attn_reduce_kernel (babyvllm/kernels/paged_attn.py:9-251).
// The single-pass work-group is decode_work_group (paged_decode_wg.h), the
// split waves are decode_stream_wave (paged_decode_stream.h); this file holds
// the kernels that launch them, the split reduce, the launch plan and the
// tuning switches.
#include "paged_decode_stream.h"

#include <algorithm>
#include <atomic>

namespace bvllm {

template <int D, int NW, int PF, bool EAGER>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  decode_work_group<D, NW, PF, EAGER>(a, blockIdx.x, smem);
}

// One streaming wave per work-group, so that a short batch's splits spread
// over every CU.
template <int D, int PF, bool NT, bool GROUP>
__global__ __launch_bounds__(64) void paged_decode_stream_kernel(DecodeArgs a, int items) {
  __shared__ __attribute__((aligned(16))) unsigned char tile[kTileBytes<D>];
  const int item = (int)blockIdx.x;
  if (item >= items) return;
  decode_stream_wave<D, PF, NT, GROUP>(a, item, tile);
}

// ---------------------------------------------------------------- the reduce
//
// Level 3 of the split merge: out = Σ_g w_g·o_g / Σ_g w_g, w_g = 2^(lse_g − M),
// M the largest lse_g, over the group results g of a (row, head), in order:
//   * groups are taken in chains of kChain consecutive groups; a chain's sums
//     are fma chains in group order: num = fma(w_g, o_g, num), den += w_g;
//   * chain sums are added in chain order, skipping chains with den == 0.
// With at most kChain groups that is one chain. When the split waves wrote one
// partial per split and the plan groups splits (level 2 not yet done), the
// reduce first folds each group's splits (GroupFold).
constexpr int kChain = 32;

// One chain's partial states for 4 dims, loaded in one round.
struct ChainRegs {
  float l[kChain];
  float4 x[kChain];
};

__device__ __forceinline__ void load_chain(ChainRegs& r, const float* lse, const float* po, int D, int s0, int n) {
#pragma unroll
  for (int k = 0; k < kChain; ++k) {
    const int s = s0 + k;
    r.l[k] = s < n ? lse[s] : kNegInf;
    r.x[k] = s < n ? *reinterpret_cast<const float4*>(po + (int64_t)s * D) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// Entries at or past `live` (a uniform count) are empty (lse -inf, output 0)
// and are not visited: an empty entry leaves the maximum and the sums
// bit-identical (weight 2^-inf = 0, fma(0, 0, x) = x), so skipping changes no
// bit, only the length of the dependent chains.
__device__ __forceinline__ float chain_max(const ChainRegs& r, int live = kChain) {
  float M = kNegInf;
#pragma unroll
  for (int k = 0; k < kChain; ++k)
    if (k < live) M = fmaxf(M, r.l[k]);
  return M;
}

// The chain's fma sums in group order.
__device__ __forceinline__ void chain_sums(const ChainRegs& r, float M, float4& num, float& den, int live = kChain) {
  num = make_float4(0.f, 0.f, 0.f, 0.f);
  den = 0.f;
#pragma unroll
  for (int k = 0; k < kChain; ++k) {
    if (k < live) {  // a guarded body, not a break: every index stays a constant (registers, not scratch)
      const float wgt = fast_exp2(r.l[k] - M);
      num.x = __builtin_fmaf(wgt, r.x[k].x, num.x);
      num.y = __builtin_fmaf(wgt, r.x[k].y, num.y);
      num.z = __builtin_fmaf(wgt, r.x[k].z, num.z);
      num.w = __builtin_fmaf(wgt, r.x[k].w, num.w);
      den += wgt;
    }
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

// At most kChain group results per (row, head): one thread per (row, head,
// 4 dims). FOLD: the workspace holds one partial per split (at most kChain of
// them), folded here into groups of kSplitGroup first. Entries past the np
// partials are empty and are not visited (folding an empty split changes
// nothing), so the dependent chains are as long as the live entries.
template <int D, bool FOLD>
__global__ __launch_bounds__(256) void decode_reduce_small_kernel(DecodeArgs a, int64_t items) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= items) return;
  const int64_t bh = t / (D / 4);
  const int d = (int)(t - bh * (D / 4)) * 4;
  const int np = a.num_partials;
  ChainRegs r;
  load_chain(r, a.part_lse + bh * np, a.part_out + bh * np * D + d, D, 0, np);
  int live = np;
  if constexpr (FOLD) {
    // Level 2 in place: group q's result replaces entry q (q < kChain / 4).
    // Guarded bodies, not breaks: every index stays a constant (registers, not scratch).
#pragma unroll
    for (int q = 0; q < kChain / kSplitGroup; ++q) {
      if (q * kSplitGroup < np) {
        GroupFold f;
        float4 gx = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < kSplitGroup; ++k) {
          const int s = q * kSplitGroup + k;
          if (s < np) {
            float wa, wb;
            group_fold_weights(f, r.l[s], wa, wb);
            gx.x = group_fold_value(gx.x, r.x[s].x, wa, wb);
            gx.y = group_fold_value(gx.y, r.x[s].y, wa, wb);
            gx.z = group_fold_value(gx.z, r.x[s].z, wa, wb);
            gx.w = group_fold_value(gx.w, r.x[s].w, wa, wb);
          }
        }
        const float inv = group_inv(f);
        r.l[q] = group_lse(f);
        r.x[q] = make_float4(gx.x * inv, gx.y * inv, gx.z * inv, gx.w * inv);
      }
    }
    live = (np + kSplitGroup - 1) / kSplitGroup;
  }
  float M = chain_max(r, live);
  if (M == kNegInf) M = 0.f;
  float4 num;
  float den;
  chain_sums(r, M, num, den, live);
  store_reduced(a, bh, d, num, den);
}

// More than kChain group results per (row, head) (written by the split
// waves, no folding): one work-group per (row, head, 32-dim slice); thread
// (chunk, q) sums chain q of the current set of chains, then the threads of
// chain 0 add the set's chain sums in order onto the running total.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeArgs a) {
  constexpr int DS = 32;          // dims per work-group
  constexpr int CH = DS / 4;      // float4 chunks per slice
  constexpr int NQ = 256 / CH;    // chains per set
  constexpr int SLICES = D / DS;
  __shared__ float red[256];
  __shared__ float4 gnum[NQ][CH];
  __shared__ float gden[NQ];

  const int64_t bh = blockIdx.x / SLICES;
  const int d0 = (blockIdx.x % SLICES) * DS;
  const int np = a.num_partials;
  const float* lse = a.part_lse + bh * np;
  const float* po = a.part_out + bh * np * D + d0;

  const int ch = threadIdx.x % CH;
  const int q = threadIdx.x / CH;
  ChainRegs r;
  float M;
  if (np <= NQ * kChain) {
    // One set: the chain loads double as the max pass.
    load_chain(r, lse, po + 4 * ch, D, q * kChain, np);
    if (ch == 0) red[q] = chain_max(r);
    __syncthreads();
    M = kNegInf;
    const int nq = (np + kChain - 1) / kChain;  // chains holding results; the others' maxima are -inf
    for (int k = 0; k < nq; ++k) M = fmaxf(M, red[k]);
  } else {
    M = kNegInf;
    for (int s = threadIdx.x; s < np; s += 256) M = fmaxf(M, lse[s]);
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
  for (int set0 = 0; set0 < np; set0 += NQ * kChain) {
    if (set0 > 0 || np > NQ * kChain) load_chain(r, lse, po + 4 * ch, D, set0 + q * kChain, np);
    float4 num;
    float den;
    chain_sums(r, M, num, den);
    gnum[q][ch] = num;
    if (ch == 0) gden[q] = den;
    __syncthreads();
    if (q == 0) {
      // Chains past the set's last result have den == 0 and would be skipped
      // below anyway; not visiting them saves a dependent LDS read each
      // (B1 x 32768, 4 of 32 chains used: 25.7-26.4 -> 24.8-25.4 us).
      const int nq = min(NQ, (np - set0 + kChain - 1) / kChain);
      for (int k = 0; k < nq; ++k) {
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

// ------------------------------------------------------------ tuning switches

// Process-wide launch choices for experiments and tests (bvllm_set_tuning);
// none changes results beyond what each knob's comment says.
static std::atomic<int> g_tuning[kTuneKnobs] = {};

int tuning(int knob) { return (knob >= 0 && knob < kTuneKnobs) ? g_tuning[knob].load(std::memory_order_relaxed) : 0; }

int set_tuning(int knob, int value) {
  if (knob < 0 || knob >= kTuneKnobs) return -1;
  return g_tuning[knob].exchange(value, std::memory_order_relaxed);
}

// ------------------------------------------------------------ the launch plan

// How a decode launch runs (the split boundaries come from the caller's plan):
//   single pass (one split): work-groups of 4 waves, bf16 output directly;
//   split, one wave per split ("split" mode): partials per split, level 2 in
//     the reduce;
//   split, one wave per group of kSplitGroup splits ("group" mode): level 2 in
//     the wave, one partial per group.
// Both split modes give the same bits. Group mode needs bps % 4 == 0 (the
// group then starts every split on a page index ≡ 0 mod 4 of the wave's
// stream); split mode folds at most kChain splits in the reduce. The default
// takes group mode when there are more than kChain splits or enough groups to
// fill the GPU (2 per CU of a 256-CU MI355X), split mode otherwise.
DecodePlan decode_plan(int32_t batch, int32_t num_kv_heads, int32_t num_splits, int32_t blocks_per_split) {
  DecodePlan p{};
  if (num_splits <= 1) {
    p.single_pass = true;
    p.partials = 0;
    return p;
  }
  p.group = (blocks_per_split % kSplitGroup == 0) ? kSplitGroup : 1;
  const int64_t groups = (num_splits + p.group - 1) / p.group;
  bool group_mode = p.group > 1 && (num_splits > kChain || (int64_t)batch * num_kv_heads * groups >= 512);
  const int forced = tuning(kTuneDecodeSplitMode);
  if (forced == 1 && (p.group == 1 || num_splits <= kChain)) group_mode = false;
  if ((forced == 2 || forced == 3) && p.group > 1) group_mode = true;
  p.splits_per_item = group_mode ? p.group : 1;
  p.partials = group_mode ? (int32_t)groups : num_splits;
  p.fold_in_reduce = !group_mode && p.group > 1;
  // Two waves per work-group: for single splits unless knob 1; for groups of
  // splits when there are at most two groups per CU (two waves per group, two
  // pages in flight each, one wave per SIMD: 1 x 32768 and 2 x 16384, 512
  // groups: 23.5 -> 21.5 and 24.1 -> 21.2 us; 4 x 4096, 256 groups: 22.0 ->
  // 18.2 us), one wave per group beyond (8 x 16384, 1024 groups: 52.8 against
  // 56.4 us on two waves; 4 x 32768, 2048 groups: 60.0 against 64.3 us).
  const int64_t group_items = (int64_t)batch * num_kv_heads * groups;
  p.pair = group_mode ? (forced == 3 || (forced != 2 && group_items <= 2 * (int64_t)device_cus())) : forced != 1;
  // Four waves per split when a split has at most 32 pages (at most 8 per wave), unless knob 4.
  p.quad = p.pair && !group_mode && blocks_per_split <= 32 && forced != 4;
  return p;
}

// The largest partial count any plan of these splits can write, whatever the
// split-mode knob says: groups only where split mode is impossible (more than
// kChain splits that group), else one per split. It sizes the workspace and
// places part_lse, so a knob changed between the size query and the launch
// cannot move either.
int32_t decode_partials(int32_t batch, int32_t num_kv_heads, int32_t num_splits, int32_t blocks_per_split) {
  (void)batch;
  (void)num_kv_heads;
  if (num_splits <= 1) return 0;
  if (blocks_per_split % kSplitGroup == 0 && num_splits > kChain) return (num_splits + kSplitGroup - 1) / kSplitGroup;
  return num_splits;
}

template <int D>
static hipError_t launch_reduce(const DecodeArgs& r, const DecodePlan& p, hipStream_t stream) {
  const int64_t groups = p.fold_in_reduce ? (r.num_partials + kSplitGroup - 1) / kSplitGroup : r.num_partials;
  if (groups <= kChain && (!p.fold_in_reduce || r.num_partials <= kChain)) {
    const int64_t items = (int64_t)r.batch * r.num_heads * (D / 4);
    const dim3 grid((unsigned)((items + 255) / 256));
    if (p.fold_in_reduce)
      hipLaunchKernelGGL((decode_reduce_small_kernel<D, true>), grid, dim3(256), 0, stream, r, items);
    else
      hipLaunchKernelGGL((decode_reduce_small_kernel<D, false>), grid, dim3(256), 0, stream, r, items);
  } else {
    if (p.fold_in_reduce) return hipErrorInvalidValue;  // excluded by decode_plan
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

// Sets a kernel's dynamic-LDS limit once per device (setting it twice, from
// racing host threads, is harmless).
template <typename K>
static hipError_t allow_lds(K* kernel, std::atomic<bool> (&done)[64], int bytes) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  if (!done[dev].load(std::memory_order_acquire)) {
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              bytes);
    if (err != hipSuccess) return err;
    done[dev].store(true, std::memory_order_release);
  }
  return hipSuccess;
}

template <int D, int PF, bool GROUP>
static hipError_t launch_stream_pf(const DecodeArgs& a, int64_t items, hipStream_t stream) {
  if (tuning(kTuneDecodeCached) == 0)
    hipLaunchKernelGGL((paged_decode_stream_kernel<D, PF, true, GROUP>), dim3((unsigned)items), dim3(64), 0,
                       stream, a, (int)items);
  else
    hipLaunchKernelGGL((paged_decode_stream_kernel<D, PF, false, GROUP>), dim3((unsigned)items), dim3(64), 0,
                       stream, a, (int)items);
  return hipGetLastError();
}

// Two pages in flight per streaming wave. (Four do not fit the register file
// next to the four states: the compiler then parks registers that in-flight
// loads still write. One, requested as soon as the previous page has landed,
// as in the single pass: B1 x 32768 24.97 against 24.92 us, and slower for
// B8's group waves, 31.2 against 30.8 us: these launches wait on latency,
// not on the DRAM.)
template <int D, bool GROUP>
static hipError_t launch_stream(const DecodeArgs& a, int64_t items, hipStream_t stream) {
  return launch_stream_pf<D, 2, GROUP>(a, items, stream);
}

template <int D>
static hipError_t launch_decode(const DecodeArgs& args, hipStream_t stream) {
  DecodeArgs a = args;
  const int64_t ncg = decode_col_groups(a);
  const DecodePlan p = decode_plan(a.batch, (int32_t)ncg, a.num_splits, a.blocks_per_split);
  a.item_order = tuning(kTuneDecodeOrder) == 1 ? 1 : 0;
  if (p.single_pass && tuning(kTuneDecodeSinglePassStream) == 0) {
    // One page in flight per wave, the next requested as soon as it has
    // landed: more requests in flight lower the rate this access pattern gets
    // from HBM (B64 x 1920: 43.0 us, against 44.5 with two pages in flight
    // requested after each page is computed, 45.1 with three, 46.9 with four;
    // 42.4 us once no load is issued past a wave's last page).
    constexpr int NW = 4;
    constexpr size_t smem = decode_lds_bytes<D, NW>();
    static_assert(smem <= 160 * 1024, "single-pass work-group LDS");
    static std::atomic<bool> done[64] = {};
    hipError_t err = allow_lds(&paged_decode_kernel<D, NW, 1, true>, done, 160 * 1024);
    if (err != hipSuccess) return err;
    const int64_t wgs = (int64_t)a.batch * decode_col_groups(a);
    if (wgs > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((paged_decode_kernel<D, NW, 1, true>), dim3((unsigned)wgs), dim3(NW * 64), smem, stream, a);
    return hipGetLastError();
  }
  a.splits_per_item = p.single_pass ? 1 : p.splits_per_item;
  a.num_partials = p.partials;
  // The workspace holds decode_partials() states per (row, head); the plan
  // (one knob read above) never asks for more.
  if (!p.single_pass && (a.part_out == nullptr || p.partials > a.ws_partials)) return hipErrorInvalidValue;
  const int64_t units = (a.num_splits + a.splits_per_item - 1) / a.splits_per_item;
  const int64_t items = (int64_t)a.batch * decode_col_groups(a) * units;
  if (items > 0x7ffffff0) return hipErrorInvalidValue;
  hipError_t err;
  if (p.quad) {
    if constexpr (D == 64) {
      err = launch_quad_vgpr(a, items, tuning(kTuneDecodeCached) == 0, stream);
    } else {
      const dim3 grid((unsigned)items);
      if (tuning(kTuneDecodeCached) == 0)
        hipLaunchKernelGGL((paged_decode_quad_kernel<D, true>), grid, dim3(256), 0, stream, a, (int)items);
      else
        hipLaunchKernelGGL((paged_decode_quad_kernel<D, false>), grid, dim3(256), 0, stream, a, (int)items);
      err = hipGetLastError();
    }
  } else if (p.pair) {
    const bool group = a.splits_per_item > 1;
    const bool nt = tuning(kTuneDecodeCached) == 0;
    err = hipErrorInvalidValue;
    if constexpr (D == 128) {  // the D = 128 split walk (every other pair walk: paged_decode_pair.hip)
      if (!group) {
        const dim3 grid((unsigned)items), block(128);
        if (nt) hipLaunchKernelGGL((paged_decode_pair_kernel<D, true, false>), grid, block, 0, stream, a, (int)items);
        else hipLaunchKernelGGL((paged_decode_pair_kernel<D, false, false>), grid, block, 0, stream, a, (int)items);
        err = hipGetLastError();
      } else {
        err = launch_pair_vgpr(a, items, group, nt, stream);
      }
    } else {
      err = launch_pair_vgpr(a, items, group, nt, stream);
    }
  } else if (a.splits_per_item > 1) {
    err = launch_stream<D, true>(a, items, stream);
  } else {
    err = launch_stream<D, false>(a, items, stream);
  }
  if (err != hipSuccess || p.single_pass) return err;
  return launch_reduce<D>(a, p, stream);
}

hipError_t paged_decode(const DecodeArgs& a, hipStream_t stream) {
  if (a.waves != 0 && a.waves != 4) return hipErrorInvalidValue;
  switch (a.head_dim) {
    case 64: return launch_decode<64>(a, stream);
    case 128: return launch_decode<128>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
