// Split (flash-decoding) paged decode on streaming waves, and the split merge.
//
// Replaces paged_decode_attn_split_kernel (babyvllm/kernels/paged_attn.py:104-213).
// A split of the plan covers pages [s·bps, (s+1)·bps) of its row (the last
// split runs to the row's last page). One wave computes one split, or a group
// of consecutive splits, as a stream of pages:
//
//   * Pages come into registers by 16-byte loads of whole 256-byte row slices
//     (the work-group path's page loads), PF pages in flight: page k + PF is
//     requested as soon as page k is consumed; K passes through the wave's
//     transpose tile into the MFMA layout, V is used from registers.
//     (Measured and rejected: staging pages in LDS by direct global -> LDS
//     loads, whose issue took a wave 3.4 us for 8 pages at batch 8; and batches
//     of four pages computed as one block, which do not fit the register file
//     next to the four states and the pages in flight.)
//   * A split keeps the 4 online-softmax states of a single-pass work-group
//     (state s takes the split's pages start+s, start+s+4, ...) and merges them
//     with merge_states' arithmetic, so a split's (o, lse) has the bits of the
//     work-group path and a row within one split matches the single pass.
//
// Split results are merged in two fixed levels, the same arithmetic wherever
// they run, so neither the launch shape nor the bucket changes the bits:
//   level 2: groups of kSplitGroup consecutive splits (when bps % 4 == 0; else
//            groups of one) fold their splits in order (GroupFold);
//   level 3: the decode reduce chains the group results (paged_decode.hip).
// Level 2 runs in the streaming wave when one wave computes a whole group (the
// plans with many splits: one partial per group is written, a quarter of the
// partial traffic), and in the reduce otherwise (few splits: one wave per
// split spreads a short batch over every CU). Empty splits (no live page)
// leave a group unchanged, and empty groups add nothing in level 3, so a graph
// launch sized for a longer bucket gives the bits of a launch sized for the
// live length.
#pragma once

#include "paged_decode_wg.h"

#include <climits>

namespace bvllm {

// Consecutive splits folded into one partial (level 2) when the plan's
// pages per split is a multiple of 4.
constexpr int kSplitGroup = 4;

// Level 2: folds the (o, lse) of a group's splits, in split order, into a
// running (M, L, A) with the online rescale: M' = max(M, lse), A = A·2^(M−M')
// + o·2^(lse−M'), L = L·2^(M−M') + 2^(lse−M'); the group's result is
// o = A · (1 / L), lse = M + log2 L (o = 0, lse = −inf when every split is
// empty). Folding an empty split (lse = −inf, o = 0) leaves (M, L, A)
// bit-identical, and a group with one non-empty split yields exactly that
// split's (o, lse).
struct GroupFold {
  float M = kNegInf;
  float L = 0.f;
};
__device__ __forceinline__ void group_fold_weights(GroupFold& f, float lse, float& wa, float& wb) {
  const float Mn = fmaxf(f.M, lse);
  if (Mn == kNegInf) {  // nothing live yet: stays empty
    wa = 1.f;
    wb = 0.f;
    return;
  }
  wa = fast_exp2(f.M - Mn);
  wb = fast_exp2(lse - Mn);
  f.L = __builtin_fmaf(f.L, wa, wb);
  f.M = Mn;
}
__device__ __forceinline__ float group_fold_value(float acc, float x, float wa, float wb) {
  return __builtin_fmaf(x, wb, acc * wa);
}
__device__ __forceinline__ float group_inv(const GroupFold& f) { return f.L > 0.f ? 1.f / f.L : 0.f; }
__device__ __forceinline__ float group_lse(const GroupFold& f) { return f.L > 0.f ? f.M + __log2f(f.L) : kNegInf; }

// One streaming decode wave: item = (row, column group, unit of
// a.splits_per_item consecutive splits), the column group being the KV head
// when G <= 16 (ColGroup); `tile` is the wave's K transpose tile
// (kTileBytes<D> bytes of LDS).
// PAIR: the item's work-group has two waves; wave w holds states 2w and 2w+1
// of each split (its pages 4k + 2w and 4k + 2w + 1), with four pages in flight
// for a single split and two for a group of splits. At the end of every split
// both waves publish their states through `xs` (kPairLdsFloats<D> floats of
// LDS, twice that with GROUP), and wave w merges elements 2w and 2w + 1 of
// every lane's accumulator vectors from the four, in order, as a single wave
// would (and folds or writes those output dims).
// QUAD (with PAIR, single splits of at most 32 pages): four waves; wave w holds
// state w (its pages 4k + w, two in flight), publishes
// it at the split's end, and merges element w of every accumulator vector from
// the four records: the same arithmetic in the same order, on a quarter of the
// pages and dims per wave.
template <int D>
constexpr int kPairRecFloats = (2 + 4 * (D / 16)) * 64;  // m, l, accumulators of one state, per lane
template <int D>
constexpr int kPairLdsFloats = 4 * kPairRecFloats<D>;

template <int D, int PF, bool NT, bool GROUP, bool PAIR = false, bool QUAD = false>
__device__ __forceinline__ void decode_stream_wave(const DecodeArgs& a, const int item, unsigned char* tile,
                                                   float* xs = nullptr) {
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int OPL = D / 4;  // output floats per lane: head n, dims VD·(4g+i) + c
  static_assert(PF == (PAIR && !GROUP && !QUAD ? 4 : 2), "pages in flight per wave");
  static_assert(!QUAD || (PAIR && !GROUP), "four waves per item: single splits only");
  const int w = PAIR ? wave_id() : 0;

  const int S = a.num_splits;
  const int spi = GROUP ? a.splits_per_item : 1;
  const int units = (S + spi - 1) / spi;
  // Column groups: the KV heads, or their 16-head parts when G > 16 (ColGroup).
  const int ncg = a.num_kv_heads * col_groups_per_kv(a.num_heads / a.num_kv_heads);
  int cg, unit, b;
  if (a.item_order == 0) {  // KV head fastest: the 4 head slices of a page are requested together
    cg = item % ncg;
    const int rest = item / ncg;
    unit = rest % units;
    b = rest / units;
  } else {  // unit fastest
    unit = item % units;
    const int rest = item / units;
    cg = rest % ncg;
    b = rest / ncg;
  }
  const ColGroup cgp = col_group(a.num_heads / a.num_kv_heads, cg);
  const int G = cgp.cols;  // heads of this column group
  const int kvh = cgp.kvh;
  const int j0 = unit * spi;
  const int j1 = min(j0 + spi, S);
  const int bps = a.blocks_per_split;
  const int p0 = j0 * bps;

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;

  // The table slice, seq_len and q are requested together (the slice index is
  // clamped into the row, so it does not wait for seq_len).
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;
  int ent = bt[min(p0 + lane, a.max_blocks - 1)];
  const int seq_len = uniform(a.seq_lens[b]);
  uint4 qb[KC];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb +
                           (int64_t)(cgp.head0 + n) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c) qb[c] = (n < G) ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }
  int n_blocks = seq_len > 0 ? (seq_len + 15) / 16 : 0;
  n_blocks = min(n_blocks, a.max_blocks);
  // The last split of the row runs to the row's last page.
  const int p_end = (j1 == S) ? n_blocks : min(j1 * bps, n_blocks);
  const int cnt = max(p_end - p0, 0);

  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) off[j] = (uint32_t)((4 * g + j) * a.c_st + VD * n);
  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;

  WaveState<D> st[4];
  auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      st[s].m = kNegInf;
      st[s].l = 0.f;
#pragma unroll
      for (int c = 0; c < VD; ++c) st[s].acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  };
  reset();

  // The accumulator elements whose output dims this wave merges: all four
  // (one wave), 2w and 2w + 1 (two waves) or w (four); o[VD·(i - i0) + c] holds
  // element i of vector c (head n, dim VD·(4g + i) + c).
  constexpr int NI = QUAD ? 1 : PAIR ? 2 : 4;
  constexpr int OPW = NI * VD;
  const int i0 = NI * w;

  // Group accumulator (level 2 in the wave; group waves only).
  float go[GROUP ? OPW : 1];
#pragma unroll
  for (int k = 0; k < (GROUP ? OPW : 1); ++k) go[k] = 0.f;
  GroupFold gf;

  const int64_t head = (int64_t)cgp.head0 + n;
  // Folds (group waves) or writes a split's (o, lse) for this wave's dims.
  auto emit = [&](int split, float (&o)[OPW], float lse) __attribute__((always_inline)) {
    if constexpr (GROUP) {
      float wa, wb;
      group_fold_weights(gf, lse, wa, wb);
#pragma unroll
      for (int k = 0; k < OPW; ++k) go[k] = group_fold_value(go[k], o[k], wa, wb);
    } else if (n < G) {
      if (S == 1) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + head * a.o_sh;
#pragma unroll
        for (int ii = 0; ii < NI; ++ii) {
          if constexpr (VD == 8) {
            uint4 pk;
            pk.x = pack_bf16x2_hw(o[VD * ii + 0], o[VD * ii + 1]);
            pk.y = pack_bf16x2_hw(o[VD * ii + 2], o[VD * ii + 3]);
            pk.z = pack_bf16x2_hw(o[VD * ii + 4], o[VD * ii + 5]);
            pk.w = pack_bf16x2_hw(o[VD * ii + 6], o[VD * ii + 7]);
            st16(dst + VD * (4 * g + i0 + ii), pk);
          } else {
            uint2 pk;
            pk.x = pack_bf16x2_hw(o[VD * ii + 0], o[VD * ii + 1]);
            pk.y = pack_bf16x2_hw(o[VD * ii + 2], o[VD * ii + 3]);
            st8(dst + VD * (4 * g + i0 + ii), pk);
          }
        }
      } else {
        const int64_t prow = ((int64_t)b * a.num_heads + head) * a.num_partials + split;
        float* dst = a.part_out + prow * D;
#pragma unroll
        for (int ii = 0; ii < NI; ++ii)
#pragma unroll
          for (int c = 0; c < VD; c += 4)
            *reinterpret_cast<float4*>(dst + VD * (4 * g + i0 + ii) + c) =
                make_float4(o[VD * ii + c], o[VD * ii + c + 1], o[VD * ii + c + 2], o[VD * ii + c + 3]);
        if (g == 0 && i0 == 0) a.part_lse[prow] = lse;
      }
    }
  };
  // Merges the 4 states of split `split` (merge_states' arithmetic, per lane)
  // and folds or writes its (o, lse). One wave: the states in registers.
  auto finish_split = [&](int split) __attribute__((always_inline)) {
    float lt[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) lt[s] = sum_across_groups(st[s].l);
    float M = kNegInf;
#pragma unroll
    for (int s = 0; s < 4; ++s) M = fmaxf(M, st[s].m);
    float L = 0.f;
    float o[OPL];
#pragma unroll
    for (int k = 0; k < OPL; ++k) o[k] = 0.f;
    if (M != kNegInf) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float wgt = fast_exp2(st[s].m - M);
        L = __builtin_fmaf(lt[s], wgt, L);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int c = 0; c < VD; ++c) o[VD * i + c] = __builtin_fmaf(st[s].acc[c][i], wgt, o[VD * i + c]);
      }
    }
    const float inv = split_inv(L);
#pragma unroll
    for (int k = 0; k < OPL; ++k) o[k] = L == 0.f ? 0.f : o[k] * inv;
    if constexpr (!PAIR) emit(split, o, split_lse(M, L));
    reset();
  };

  // PAIR: both waves publish their two states (records 2w and 2w + 1 of LDS
  // buffer xb, global states 2w and 2w + 1) and restart them; after one
  // barrier wave w merges elements i0, i0 + 1 of every lane's accumulator
  // vectors from the four records, in state order, and folds or writes them.
  // QUAD: each of the four waves publishes its one state (record w) and
  // merges element w.
  auto pair_finish = [&](int xb, int split) __attribute__((always_inline)) {
    float* xbase = xs + xb * kPairLdsFloats<D>;
    constexpr int SPW = QUAD ? 1 : 2;  // states per wave
#pragma unroll
    for (int s2 = 0; s2 < SPW; ++s2) {
      float* rec = xbase + (SPW * w + s2) * kPairRecFloats<D>;
      rec[lane] = st[s2].m;
      rec[64 + lane] = st[s2].l;
#pragma unroll
      for (int c = 0; c < VD; ++c) *reinterpret_cast<f32x4_t*>(rec + 128 + (c * 64 + lane) * 4) = st[s2].acc[c];
    }
    reset();
    __syncthreads();
    // Every read of the four records is issued before any is used: one wait
    // (inside a branch around the sums they went out one or two at a time,
    // each waited for).
    float mv[4], lraw[4];
    float xr[4][VD][NI];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      mv[s] = xbase[s * kPairRecFloats<D> + lane];
      lraw[s] = xbase[s * kPairRecFloats<D> + 64 + lane];
      const float* racc = xbase + s * kPairRecFloats<D> + 128 + i0;
#pragma unroll
      for (int c = 0; c < VD; ++c) {
        if constexpr (NI == 2) {
          const float2 x2 = *reinterpret_cast<const float2*>(racc + (c * 64 + lane) * 4);
          xr[s][c][0] = x2.x;
          xr[s][c][1] = x2.y;
        } else {
          xr[s][c][0] = racc[(c * 64 + lane) * 4];
        }
      }
    }
    float lt[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) lt[s] = sum_across_groups(lraw[s]);
    float M = kNegInf;
#pragma unroll
    for (int s = 0; s < 4; ++s) M = fmaxf(M, mv[s]);
    float L = 0.f;
    float o[OPW];
#pragma unroll
    for (int k = 0; k < OPW; ++k) o[k] = 0.f;
    // No branch around the sums (a branch let the compiler sink the reads into
    // it): with every state empty (M = -inf) the weights are 0 and so are
    // the accumulators and sums, so L and o stay +0 as they would unsummed
    // (B1 x 32768: 21.0 -> 20.7 us, B8 x 1920: 14.37 -> 14.20 us).
    const bool live = M != kNegInf;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float wgt = live ? fast_exp2(mv[s] - M) : 0.f;
      L = __builtin_fmaf(lt[s], wgt, L);
#pragma unroll
      for (int c = 0; c < VD; ++c) {
#pragma unroll
        for (int ii = 0; ii < NI; ++ii) o[VD * ii + c] = __builtin_fmaf(xr[s][c][ii], wgt, o[VD * ii + c]);
      }
    }
    const float inv = split_inv(L);
#pragma unroll
    for (int k = 0; k < OPW; ++k) o[k] = L == 0.f ? 0.f : o[k] * inv;
    emit(split, o, split_lse(M, L));
  };
  int xb = 0;  // PAIR with GROUP: the exchange buffers alternate, so no wave
               // overwrites a record the other has not read (a barrier lies between)

  int cur = j0;  // split whose states are open
  // Item-relative page index where split cur + 1 starts (none past the unit).
  int next_start = (cur + 1 < j1) ? bps : INT_MAX;
  bool any = false;  // a page of split cur was processed

  // Pages are taken four at a time (page k + i into state i), PF in flight;
  // loads are issued for clamped page indices (in bounds), and pages past the
  // chunk's end are skipped (a fully masked page would leave its state
  // bit-identical anyway).
  for (int base = 0; base < cnt; base += 64) {
    const int here = min(64, cnt - base);
    if (base > 0) ent = bt[min(p0 + base + lane, a.max_blocks - 1)];
    const int slot_ent = min(max(ent, 0), a.num_pages - 1);
    auto phys = [&](int k) -> int64_t { return (int64_t)__builtin_amdgcn_readlane(slot_ent, k); };
    PageRegs<D> r[PF];
    if constexpr (PAIR && GROUP) {
      // A group of splits on two waves: two pages in flight per wave, page
      // k + 4 requested once page k is computed. The wave's pages in order:
      // q = 4j + 2w + i for ring slot i, state i (global state 2w + i).
      // (Four in flight, as in split mode, put 32 MB of requests in flight at
      // B1 x 32768 and ran it in 24.3 us against 21.2.)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int64_t p = phys(min(2 * w + i, here - 1)) * a.c_sb;
        load_page<D, NT>(r[i], kc + p, vc + p, off);
      }
      // At a split's first page: the split that ended is merged and folded.
      auto new_split = [&](int quad) __attribute__((always_inline)) {
        if (quad < here && base + quad == next_start) {
          pair_finish(xb, cur);
          xb ^= 1;
          ++cur;
          next_start = (cur + 1 < j1) ? next_start + bps : INT_MAX;
          any = false;
        }
      };
      int k = 0;
      for (; k + 4 < here; k += 4) {
        new_split(k);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          wait_page<kLoadsPerPage, D>(r[i]);
          const int q = k + 2 * w + i;
          if (q < here)
            process_page<D>(st[i], r[i], qb, tile, n, g, (p0 + base + q) * 16 + 4 * g, seq_len, a.scale_log2);
          const int64_t pn = phys(min(q + 4, here - 1)) * a.c_sb;
          load_page<D, NT>(r[i], kc + pn, vc + pn, off);
        }
        any = true;
      }
      // The last four pages: no load past them, and slot i waits for itself only.
      new_split(k);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (i == 0) wait_page<kLoadsPerPage, D>(r[0]);
        else wait_page<0, D>(r[1]);
        const int q = k + 2 * w + i;
        if (q < here)
          process_page<D>(st[i], r[i], qb, tile, n, g, (p0 + base + q) * 16 + 4 * g, seq_len, a.scale_log2);
      }
      any = true;
      continue;
    }
    if constexpr (QUAD) {
      // Split mode on four waves, two pages in flight per wave: the wave's
      // pages in order are q = 8j + 4i + w for ring slot i, all of state w.
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int64_t p = phys(min(4 * i + w, here - 1)) * a.c_sb;
        load_page<D, NT>(r[i], kc + p, vc + p, off);
      }
      int k = 0;
      for (; k + 8 < here; k += 8) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
          wait_page<(PF - 1) * kLoadsPerPage, D>(r[i]);
          const int q = k + 4 * i + w;
          if (q < here)
            process_page<D>(st[0], r[i], qb, tile, n, g, (p0 + base + q) * 16 + 4 * g, seq_len, a.scale_log2);
          const int64_t pn = phys(min(q + 8, here - 1)) * a.c_sb;
          load_page<D, NT>(r[i], kc + pn, vc + pn, off);
        }
      }
      // The last eight pages: no load past them, and slot i waits for itself only.
      wait_page<kLoadsPerPage, D>(r[0]);
      if (k + w < here)
        process_page<D>(st[0], r[0], qb, tile, n, g, (p0 + base + k + w) * 16 + 4 * g, seq_len, a.scale_log2);
      wait_page<0, D>(r[1]);
      if (k + 4 + w < here)
        process_page<D>(st[0], r[1], qb, tile, n, g, (p0 + base + k + 4 + w) * 16 + 4 * g, seq_len, a.scale_log2);
      continue;
    }
    if constexpr (PAIR) {
      // Split mode on two waves, four pages in flight per wave: the wave's
      // pages in order are q = 8j + 4(i/2) + 2w + (i mod 2) for ring slot i,
      // state i mod 2 (global state 2w + i mod 2).
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int64_t p = phys(min(4 * (i >> 1) + 2 * w + (i & 1), here - 1)) * a.c_sb;
        load_page<D, NT>(r[i], kc + p, vc + p, off);
      }
      int k = 0;
      for (; k + 8 < here; k += 8) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
          const int quad = k + 4 * (i >> 1);  // first page of the 4-page block of slot i
          wait_page<(PF - 1) * kLoadsPerPage, D>(r[i]);
          const int q = quad + 2 * w + (i & 1);
          if (q < here)
            process_page<D>(st[i & 1], r[i], qb, tile, n, g, (p0 + base + q) * 16 + 4 * g, seq_len, a.scale_log2);
          const int64_t pn = phys(min(q + 8, here - 1)) * a.c_sb;
          load_page<D, NT>(r[i], kc + pn, vc + pn, off);
          if ((i & 1) == 1 && quad < here) any = true;
        }
      }
      // The last eight pages (all of them when the chunk has at most eight, as
      // in a split of 8 pages): no load past them, and slot i waits for itself
      // only (B8 x 1920: 15.6 -> 14.8 us).
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int quad = k + 4 * (i >> 1);
        if (i == 0) wait_page<3 * kLoadsPerPage, D>(r[0]);
        else if (i == 1) wait_page<2 * kLoadsPerPage, D>(r[1]);
        else if (i == 2) wait_page<kLoadsPerPage, D>(r[2]);
        else wait_page<0, D>(r[3]);
        const int q = quad + 2 * w + (i & 1);
        if (q < here)
          process_page<D>(st[i & 1], r[i], qb, tile, n, g, (p0 + base + q) * 16 + 4 * g, seq_len, a.scale_log2);
        if ((i & 1) == 1 && quad < here) any = true;
      }
      continue;
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int64_t p = phys(min(i, here - 1)) * a.c_sb;
      load_page<D, NT>(r[i], kc + p, vc + p, off);
    }
    for (int k = 0; k < here; k += 4) {
      if constexpr (GROUP) {
        if (base + k == next_start) {  // a new split of the unit starts at this page
          finish_split(cur);
          ++cur;
          next_start = (cur + 1 < j1) ? next_start + bps : INT_MAX;
          any = false;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wait_page<(PF - 1) * kLoadsPerPage, D>(r[i % PF]);
        const int page = p0 + base + k + i;
        if (k + i < here)
          process_page<D>(st[i], r[i % PF], qb, tile, n, g, page * 16 + 4 * g, seq_len, a.scale_log2);
        const int64_t pn = phys(min(k + i + PF, here - 1)) * a.c_sb;
        load_page<D, NT>(r[i % PF], kc + pn, vc + pn, off);
      }
      any = true;
    }
    // Drain: the loads issued past the end must land before their registers
    // are reused.
#pragma unroll
    for (int i = 0; i < PF; ++i) wait_page<0, D>(r[i]);
  }
  // The split holding the unit's last pages (for a unit of one split, also
  // when it has no page: its partial is written as empty). Both waves of a
  // pair agree on `any`: it follows the 4-page blocks, not the pages each
  // wave computed.
  if (any || !GROUP) {
    if constexpr (PAIR) pair_finish(xb, cur);
    else finish_split(cur);
  }

  if (GROUP && n < G) {
    const int64_t prow = ((int64_t)b * a.num_heads + head) * a.num_partials + unit;
    float* dst = a.part_out + prow * D;
    const float ginv = group_inv(gf);
#pragma unroll
    for (int ii = 0; ii < NI; ++ii)
#pragma unroll
      for (int c = 0; c < VD; c += 4)
        *reinterpret_cast<float4*>(dst + VD * (4 * g + i0 + ii) + c) =
            make_float4(go[VD * ii + c] * ginv, go[VD * ii + c + 1] * ginv, go[VD * ii + c + 2] * ginv,
                        go[VD * ii + c + 3] * ginv);
    if (g == 0 && i0 == 0) a.part_lse[prow] = group_lse(gf);
  }
}

// Two waves per split (four pages in flight each) or per group of splits
// (two). Each specialization is instantiated by one translation unit only:
// paged_decode_pair.hip (built with the MFMA accumulators in VGPRs) launches
// the group walks and the D = 64 split walk, paged_decode.hip the D = 128
// split walk.
template <int D, bool NT, bool GROUP>
__global__ __launch_bounds__(128) void paged_decode_pair_kernel(DecodeArgs a, int items) {
  __shared__ __attribute__((aligned(16))) unsigned char tile[2 * kTileBytes<D>];
  __shared__ __attribute__((aligned(16))) float xs[(GROUP ? 2 : 1) * kPairLdsFloats<D>];
  const int item = (int)blockIdx.x;
  if (item >= items) return;
  decode_stream_wave<D, GROUP ? 2 : 4, NT, GROUP, true>(a, item, tile + wave_id() * kTileBytes<D>, xs);
}

// Four waves per single split of at most 32 pages (one state each, two pages
// in flight): B8 x 1920 (15 splits of 8 pages) 14.3 -> 13.9 us, config 1 (4 of
// 8) 11.13 -> 10.85 us, B8 x 4096 (32 of 8) 25.0 -> 23.0 us, B16 x 1920 (8 of
// 16) 19.3 -> 18.6 us, B16 x 4096 (16 of 16) 34.1 -> 31.5 us, B32 x 1920 (4 of
// 32) 29.3 -> 28.8 us, B24 x 4096 (8 of 32) 47.2 -> 40.9 us per layer against
// two waves per split. D = 128
// is instantiated by paged_decode.hip, D = 64 by paged_decode_pair.hip (with
// VGPR accumulators: config 1 10.76 -> 10.68 us; D = 128 that way 13.97 ->
// 14.04 us at B8).
template <int D, bool NT>
__global__ __launch_bounds__(256) void paged_decode_quad_kernel(DecodeArgs a, int items) {
  __shared__ __attribute__((aligned(16))) unsigned char tile[4 * kTileBytes<D>];
  __shared__ __attribute__((aligned(16))) float xs[kPairLdsFloats<D>];
  const int item = (int)blockIdx.x;
  if (item >= items) return;
  decode_stream_wave<D, 2, NT, false, true, true>(a, item, tile + wave_id() * kTileBytes<D>, xs);
}

// Launches paged_decode_pair_kernel<D, nt, group> for the specializations
// paged_decode_pair.hip holds (group walks, and split walks at D = 64).
hipError_t launch_pair_vgpr(const DecodeArgs& a, int64_t items, bool group, bool nt, hipStream_t stream);
// Launches paged_decode_quad_kernel<64, nt> (held by paged_decode_pair.hip).
hipError_t launch_quad_vgpr(const DecodeArgs& a, int64_t items, bool nt, hipStream_t stream);

}  // namespace bvllm
