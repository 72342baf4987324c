// The paged decode work-group: device code shared by the decode kernel
// (paged_decode.hip) and the prefill kernel, which runs the single-query
// sequences of a mixed step with it.
//
// Paged decode attention: one query token per sequence against its paged K/V,
// with the flash-decoding split (partial softmax per split + LSE reduce).
//
// Replaces paged_decode_attn_kernel, paged_decode_attn_split_kernel and
// paged_decode_attn_reduce_kernel (babyvllm/kernels/paged_attn.py:9-251).
//
// Work-group = (sequence b, KV head, split). Its NW waves walk the split's
// pages interleaved (wave w takes pages start+w, start+w+NW, ...), each with a
// private online-softmax state, and merge the NW states in LDS in wave order.
// The page→wave assignment depends only on the split's first page and NW, so
// a row that fits in one split gives the same bits whether the launch is the
// single-pass one (one split) or a split one.
//
// Loads: a page of one KV head is 16 token rows of D·2 bytes at a 1 KB stride
// (7B shape). Both K and V are fetched as 4 whole rows per instruction (lane
// (n + 16g) reads row 4g+j, bytes 2·(D/16)·n, j < 4), i.e. full 128-byte lines.
// V is consumed in that layout; K is transposed through a wave-private LDS
// tile (write in the load layout, read in the MFMA layout, no barrier: a
// wave's LDS operations complete in order).
//
// Per page (16 tokens) and wave, both products run on bf16 MFMA:
//   Sᵀ[16 tok × 16 col] = K[16 tok × D] · Qᵀ[D × 16 col]   (D/32 × mfma 16x16x32)
//     col n < G is query head kvh·G + n (the GQA group), the rest is zero padding.
//     Lane (n + 16g) reads K row n, dims 8(4c+g)..+8 for c < D/32 from the tile;
//     the result lane (n + 16g) holds S[head n][token 4g+i], i < 4.
//   Oᵀ[D × 16 col] += Vᵀ[D × 16 tok] · Pᵀ[16 tok × 16 col]  (D/16 × mfma 16x16x16)
//     P comes straight from the Sᵀ registers (same lane layout as the B operand);
//     MFMA c takes element c of the lane's 4 V rows, so its output row r is dim
//     (D/16)·r + c. Lane (n + 16g) ends up holding O[head n][dims (D/4)·g .. +D/4).
// The softmax state (max, sum) of head n lives in lanes n, n+16, n+32, n+48, so
// the rescale of O by exp(m_old − m_new) needs no cross-lane traffic.
#pragma once

#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

#include <type_traits>

namespace bvllm {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
// D/16 bf16 of one row, as a register vector (usable as an asm operand).
template <int D>
using RowSlice = typename std::conditional<(D / 16) == 8, u32x4_t, u32x2_t>::type;

template <int D>
struct PageRegs {
  RowSlice<D> k[4];  // K rows 4g..4g+3, dims (D/16)·n ..
  RowSlice<D> v[4];  // V rows 4g..4g+3, dims (D/16)·n ..
};

// Page loads are issued as inline-asm global loads with explicit waits, so a
// wave keeps PF pages in flight across its loop: the compiler's own waitcnt
// insertion drains every outstanding load at a loop header, which would
// serialise memory latency and compute. wait_page<N>() waits until at most N
// loads are outstanding and is tied to the page's registers, so no use of
// them can move above it. Every asm load is followed, before its registers go
// dead, by a wait that covers it (the loop's drain).
// The loads carry the nontemporal hint: each KV byte is read once per call, and
// streaming it past the caches lifts the read rate of this access pattern by
// about 12% on MI355X (6.37 vs 5.61 TB/s measured without compute).
template <int D>
__device__ __forceinline__ void gload(RowSlice<D>& r, const uint16_t* base, uint32_t off_elems) {
  const uint32_t off = off_elems * 2;
  if constexpr (D / 16 == 8) asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(r) : "v"(off), "s"(base));
  else asm volatile("global_load_dwordx2 %0, %1, %2 nt" : "=v"(r) : "v"(off), "s"(base));
}

template <int D>
__device__ __forceinline__ void load_page(PageRegs<D>& r, const uint16_t* kbase, const uint16_t* vbase,
                                          const uint32_t (&off)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) gload<D>(r.k[j], kbase, off[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) gload<D>(r.v[j], vbase, off[j]);
}

constexpr int kLoadsPerPage = 8;

template <int N, int D>
__device__ __forceinline__ void wait_page(PageRegs<D>& r) {
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(r.k[0]), "+v"(r.k[1]), "+v"(r.k[2]), "+v"(r.k[3]),
                 "+v"(r.v[0]), "+v"(r.v[1]), "+v"(r.v[2]), "+v"(r.v[3])
               : "n"(N));
}

template <int D>
struct WaveState {
  float m;              // running max of head (lane & 15), log2 units
  float l;              // this lane's share of the running sum
  f32x4_t acc[D / 16];  // acc[c][i] = O[head][(D/16)·(4g+i) + c]
};

// One page of the online softmax. Tokens at or past tok_limit are masked: their
// scores become -inf and their V rows are replaced by zeros where they are used
// (unwritten slots may hold NaN, and 0·NaN would poison the PV product). The
// masking is branch-free so that the loads of the pages in flight stay in flight.
template <int D>
__device__ __forceinline__ void process_page(WaveState<D>& st, const PageRegs<D>& r, const uint4 (&qb)[D / 32],
                                             unsigned char* tile, int n, int g,
                                             int tok0, int tok_limit, float scale_log2) {
  constexpr int VD = D / 16;
  constexpr int PITCH = 2 * D + 16;  // bytes; the pad keeps 16-row column reads conflict-free
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<RowSlice<D>*>(tile + (4 * g + j) * PITCH + 2 * VD * n) = r.k[j];
  asm volatile("" ::: "memory");
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < D / 32; ++c) s = mfma_16x16x32(ld16(tile + n * PITCH + 16 * (4 * c + g)), qb[c], s);
  asm volatile("" ::: "memory");

  bool live[4];
  float sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    live[i] = tok0 + i < tok_limit;
    sv[i] = live[i] ? s[i] * scale_log2 : kNegInf;
  }
  float mx = fmax_prop(fmax_prop(sv[0], sv[1]), fmax_prop(sv[2], sv[3]));
  mx = max_across_groups(mx);
  const float m_new = fmax_prop(st.m, mx);
  // A page with no live token leaves the state bit-identical: m_new == m,
  // alpha == 1 and p == 0. While no live token has been seen (m_new == -inf,
  // e.g. a padding page that opens a split's state) 0 stands in for the max,
  // so that alpha and p are 0 instead of exp2(-inf - -inf) = NaN.
  const float m_ref = m_new == kNegInf ? 0.f : m_new;
  const float alpha = fast_exp2(st.m - m_ref);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_ref);
  st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  st.m = m_new;
  if (!wave_all_one(alpha)) {  // x·1 == x: skipping is exact
#pragma unroll
    for (int c = 0; c < VD; ++c) st.acc[c] *= alpha;
  }

  uint2 pb;
  pb.x = pack_bf16x2_hw(p[0], p[1]);
  pb.y = pack_bf16x2_hw(p[2], p[3]);
  constexpr int VW = VD / 2;  // dwords per V row slice
  uint32_t vv[4][VW];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int x = 0; x < VW; ++x) vv[j][x] = live[j] ? r.v[j][x] : 0u;
  }
#pragma unroll
  for (int c = 0; c < VD; ++c) {
    uint2 va;
    va.x = pick_halves(vv[0][c / 2], vv[1][c / 2], c & 1);
    va.y = pick_halves(vv[2][c / 2], vv[3][c / 2], c & 1);
    st.acc[c] = mfma_16x16x16(va, pb, st.acc[c]);
  }
}

// Bytes of one wave's K transpose tile: 16 rows of D bf16 + 16 bytes of pad.
template <int D>
constexpr int kTileBytes = 16 * (2 * D + 16);

// Saves a wave's final state as a merge record: m[16], l[16], acc[G][D]
// (row h of acc = head h of the group, un-normalised).
template <int D>
__device__ __forceinline__ void save_state(float* rec, const WaveState<D>& st, float l_tot, int G, int n, int g) {
  constexpr int VD = D / 16;
  constexpr int OD = D / 4;
  if (g == 0) {
    rec[n] = st.m;
    rec[16 + n] = l_tot;
  }
  if (n < G) {
    float* dst = rec + 32 + n * D + OD * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int c = 0; c < VD; ++c) dst[VD * i + c] = st.acc[c][i];
    }
  }
}

// Merges the NS wave states of one split in wave order (record s at
// rec + s·rec_stride) and writes the bf16 output row (one split) or the split's
// fp32 partial output and LSE. Thread `tid` of `nthreads` handles 4
// consecutive dims of one head at a time.
template <int D, int NS>
__device__ __forceinline__ void merge_states(const DecodeArgs& a, const float* rec, int rec_stride, int G, int b,
                                             int row, int kvh, int split, int tid, int nthreads) {
  const int total4 = G * D / 4;
  for (int e = tid; e < total4; e += nthreads) {
    const int h = (e * 4) / D;
    const int d = (e * 4) % D;
    float M = kNegInf;
#pragma unroll
    for (int s = 0; s < NS; ++s) M = fmaxf(M, rec[s * rec_stride + h]);
    float L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    if (M != kNegInf) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float* ws = rec + s * rec_stride;
        const float wgt = fast_exp2(ws[h] - M);
        L = __builtin_fmaf(ws[16 + h], wgt, L);
        const float4 x = *reinterpret_cast<const float4*>(ws + 32 + h * D + d);
        A.x = __builtin_fmaf(x.x, wgt, A.x);
        A.y = __builtin_fmaf(x.y, wgt, A.y);
        A.z = __builtin_fmaf(x.z, wgt, A.z);
        A.w = __builtin_fmaf(x.w, wgt, A.w);
      }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float4 o = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
    if (L == 0.f) o = make_float4(0.f, 0.f, 0.f, 0.f);
    const int head = kvh * G + h;
    if (a.num_splits == 1) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.o_sb + (int64_t)head * a.o_sh + d;
      uint2 pk;
      pk.x = pack_bf16x2_hw(o.x, o.y);
      pk.y = pack_bf16x2_hw(o.z, o.w);
      st8(dst, pk);
    } else {
      const int64_t prow = ((int64_t)b * a.num_heads + head) * a.num_splits + split;
      *reinterpret_cast<float4*>(a.part_out + prow * D + d) = o;
      if (d == 0) a.part_lse[prow] = (L > 0.f) ? M + __log2f(L) : kNegInf;
    }
  }
}

// LDS bytes one decode work-group uses: NW K transpose tiles, then NW merge
// records of 32 + G·D floats.
template <int D, int NW>
constexpr size_t decode_lds_bytes(int G) {
  return (size_t)NW * kTileBytes<D> + (size_t)NW * (32 + G * D) * sizeof(float);
}

// One decode work-group: (sequence, KV head, group of a.splits_per_wg
// consecutive splits) = wg, with NW waves and `smem` pointing at
// decode_lds_bytes<D, NW>(G) bytes of LDS. Each split's state is computed
// exactly as a work-group of its own would (waves interleave the split's pages
// from its first page, merge in wave order), so the bits do not depend on
// splits_per_wg; the pages of the group's next split are already in flight
// while a split is merged. splits_per_wg > 1 requires blocks_per_split % NW == 0,
// so that wave w's pages of consecutive full splits continue one progression
// (first page + w, stride NW) and all waves finish a full split together.
template <int D, int NW, int PF>
__device__ __forceinline__ void decode_work_group(const DecodeArgs& a, const int wg, float* smem) {
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;

  const int G = a.num_heads / a.num_kv_heads;
  const int gps = a.splits_per_wg;
  const int n_groups = (a.num_splits + gps - 1) / gps;
  const int grp = wg % n_groups;
  const int bk = wg / n_groups;
  const int kvh = bk % a.num_kv_heads;
  const int b = bk / a.num_kv_heads;
  const int j0 = grp * gps;
  const int j1 = min(j0 + gps, a.num_splits);  // splits [j0, j1)

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;
  const int w = wave_id();

  int row = b;  // q / out row
  int seq_len;
  if (a.query_start_loc != nullptr) {
    row = uniform(a.query_start_loc[b]);
    if (uniform(a.query_start_loc[b + 1]) - row != 1) return;  // left to the prefill kernel
    seq_len = min(uniform(a.seq_lens[b]), uniform(a.context_lens[b]) + 1);
  } else {
    seq_len = uniform(a.seq_lens[b]);
  }
  int n_blocks = seq_len > 0 ? (seq_len + 15) / 16 : 0;
  n_blocks = min(n_blocks, a.max_blocks);
  const int bps = a.blocks_per_split;
  const int start = j0 * bps;
  // The last split of the row runs to the row's last page.
  const int end = (j1 == a.num_splits) ? n_blocks : min(j1 * bps, n_blocks);
  const int ppw = bps / NW;  // pages of a full split per wave (splits_per_wg > 1)

  // Qᵀ operand: lane (n + 16g), chunk c -> q[b][kvh·G + n][8(4c+g) .. +8).
  uint4 qb[KC];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)row * a.q_sb +
                           (int64_t)(kvh * G + n) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c) qb[c] = (n < G) ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }

  WaveState<D> st;
  auto reset = [&]() {
    st.m = kNegInf;
    st.l = 0.f;
#pragma unroll
    for (int c = 0; c < VD; ++c) st.acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  reset();

  // Merge records (m[16], l[16], acc[G][D] per wave) follow the NW K tiles.
  const int wstride = 32 + G * D;
  float* merge = smem + NW * kTileBytes<D> / 4;
  // Merges the NW wave states of split j in wave order and writes its result.
  // Every wave calls it the same number of times.
  auto finish_split = [&](int j) {
    save_state<D>(merge + w * wstride, st, sum_across_groups(st.l), G, n, g);
    __syncthreads();
    merge_states<D, NW>(a, merge, wstride, G, b, row, kvh, j, threadIdx.x, NW * 64);
    __syncthreads();  // records are rewritten by the next split
    reset();
  };

  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) off[j] = (uint32_t)((4 * g + j) * a.c_st + VD * n);
  unsigned char* tile = reinterpret_cast<unsigned char*>(smem) + w * kTileBytes<D>;

  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  const int first = start + w;
  const int cnt = (end > first) ? (end - first + NW - 1) / NW : 0;
  int j_cur = j0;  // split the wave state belongs to
  // Lane k holds the table entry of this wave's page number base + k. The first
  // slice is requested together with seq_len and q (its index is clamped into
  // the row, so it does not wait for seq_len); entries past the row are unused.
  int ent = bt[min(first + NW * lane, a.max_blocks - 1)];
  for (int base = 0; base < cnt; base += 64) {
    const int here = min(64, cnt - base);
    if (base > 0) ent = bt[min(first + NW * (base + lane), a.max_blocks - 1)];
    const int slot_ent = min(max(ent, 0), a.num_pages - 1);
    auto phys = [&](int k) -> int64_t { return (int64_t)__builtin_amdgcn_readlane(slot_ent, k); };

    // PF pages in flight per wave: page k+PF is requested as soon as page k is
    // consumed. Loads are issued unconditionally (page index clamped into the
    // wave's range) and the page count is padded to a multiple of PF with fully
    // masked pages, so every wait counts exactly PF-1 younger pages.
    PageRegs<D> r[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int64_t p = phys(min(i, here - 1)) * a.c_sb;
      load_page<D>(r[i], kc + p, vc + p, off);
    }
    const int padded = (here + PF - 1) / PF * PF;
    for (int k = 0; k < padded; k += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        wait_page<(PF - 1) * kLoadsPerPage, D>(r[i]);
        const int idx = base + k + i;
        const int page = first + NW * idx;
        const int limit = (k + i < here) ? seq_len : 0;
        process_page<D>(st, r[i], qb, tile, n, g, page * 16 + 4 * g, limit, a.scale_log2);
        const int64_t pn = phys(min(k + i + PF, here - 1)) * a.c_sb;
        load_page<D>(r[i], kc + pn, vc + pn, off);
        // End of a full split that is not the group's last: every wave is here.
        if (gps > 1 && k + i < here && (idx + 1) % ppw == 0 && j_cur < j1 - 1 && (j_cur + 1) * bps <= n_blocks) {
          finish_split(j_cur);
          ++j_cur;
        }
      }
    }
    // Drain: the loads issued for pages past the end must land before their
    // registers are reused.
#pragma unroll
    for (int i = 0; i < PF; ++i) wait_page<0, D>(r[i]);
  }
  // The split holding the wave's last pages, then the group's splits that the
  // row does not reach (zero output, -inf LSE).
  for (; j_cur < j1; ++j_cur) finish_split(j_cur);
}

// One split of one (sequence, KV head) on a single wave, for plans with many
// short splits. The wave keeps the NW = 4 states that the waves of a
// decode_work_group would keep (state s takes the split's pages start + s,
// start + s + 4, ...), computes each page with the same process_page, and
// merges the four states in registers with merge_states' arithmetic (max in
// state order, then fma chains in state order), so the bits equal those of
// decode_work_group for the same split. No LDS merge records and no
// barriers: the wave needs no other wave. `tile` is the wave's private K
// transpose tile (kTileBytes<D> bytes).
template <int D, int PF>
__device__ __forceinline__ void decode_split_wave(const DecodeArgs& a, const int item, unsigned char* tile) {
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int NS = 4;  // the states of a 4-wave work-group
  static_assert(PF == 2 || PF == 4, "pages in flight per wave");

  const int G = a.num_heads / a.num_kv_heads;
  const int split = item % a.num_splits;
  const int bk = item / a.num_splits;
  const int kvh = bk % a.num_kv_heads;
  const int b = bk / a.num_kv_heads;

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;

  const int seq_len = uniform(a.seq_lens[b]);
  int n_blocks = seq_len > 0 ? (seq_len + 15) / 16 : 0;
  n_blocks = min(n_blocks, a.max_blocks);
  const int start = split * a.blocks_per_split;
  // The last split of the row runs to the row's last page.
  const int end = (split == a.num_splits - 1) ? n_blocks : min(start + a.blocks_per_split, n_blocks);
  const int cnt = max(end - start, 0);

  uint4 qb[KC];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb +
                           (int64_t)(kvh * G + n) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c) qb[c] = (n < G) ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }

  WaveState<D> st[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    st[s].m = kNegInf;
    st[s].l = 0.f;
#pragma unroll
    for (int c = 0; c < VD; ++c) st[s].acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) off[j] = (uint32_t)((4 * g + j) * a.c_st + VD * n);
  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  // Pages are taken four at a time (one per state), PF in flight; loads are
  // issued for clamped page indices, and pages past the split's end are
  // skipped (a fully masked page would leave its state bit-identical anyway).
  for (int base = 0; base < cnt; base += 64) {
    const int here = min(64, cnt - base);
    const int ent = bt[min(start + base + lane, a.max_blocks - 1)];
    const int slot_ent = min(max(ent, 0), a.num_pages - 1);
    auto phys = [&](int k) -> int64_t { return (int64_t)__builtin_amdgcn_readlane(slot_ent, k); };
    PageRegs<D> r[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int64_t p = phys(min(i, here - 1)) * a.c_sb;
      load_page<D>(r[i], kc + p, vc + p, off);
    }
    const int padded = (here + NS - 1) / NS * NS;
    for (int k = 0; k < padded; k += NS) {
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        wait_page<(PF - 1) * kLoadsPerPage, D>(r[i % PF]);
        const int page = start + base + k + i;
        if (k + i < here)
          process_page<D>(st[i], r[i % PF], qb, tile, n, g, page * 16 + 4 * g, seq_len, a.scale_log2);
        const int64_t pn = phys(min(k + i + PF, here - 1)) * a.c_sb;
        load_page<D>(r[i % PF], kc + pn, vc + pn, off);
      }
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) wait_page<0, D>(r[i]);
  }

  // merge_states' arithmetic, per lane: head n, dims (D/16)·(4g+i) + c.
  float lt[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) lt[s] = sum_across_groups(st[s].l);
  float M = kNegInf;
#pragma unroll
  for (int s = 0; s < NS; ++s) M = fmaxf(M, st[s].m);
  float L = 0.f;
  f32x4_t A[VD];
#pragma unroll
  for (int c = 0; c < VD; ++c) A[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (M != kNegInf) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float wgt = fast_exp2(st[s].m - M);
      L = __builtin_fmaf(lt[s], wgt, L);
#pragma unroll
      for (int c = 0; c < VD; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) A[c][i] = __builtin_fmaf(st[s].acc[c][i], wgt, A[c][i]);
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (n >= G) return;
  const int head = kvh * G + n;
  const int64_t prow = ((int64_t)b * a.num_heads + head) * a.num_splits + split;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float o[VD];
#pragma unroll
    for (int c = 0; c < VD; ++c) o[c] = L == 0.f ? 0.f : A[c][i] * inv;
    float* dst = a.part_out + prow * D + VD * (4 * g + i);
    if constexpr (VD == 8) {
      *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
    } else {
      *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
  if (g == 0) a.part_lse[prow] = (L > 0.f) ? M + __log2f(L) : kNegInf;
}

}  // namespace bvllm
