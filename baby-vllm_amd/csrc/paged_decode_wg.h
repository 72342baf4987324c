// The paged decode work-group: device code shared by the decode kernel
// (paged_decode.hip) and the prefill kernel, which runs the single-query
// sequences of a mixed step with it.
//
// Replaces paged_decode_attn_kernel (babyvllm/kernels/paged_attn.py:9-101),
// the single-pass decode; the page math (page_scores, page_softmax_pv) is
// shared with the split launches.
//
// Work-group = (sequence b, KV head) of a single-pass launch (with more than 16
// query heads per KV head, (sequence b, column group): see ColGroup). Its NW = 4 waves
// walk the row's pages interleaved (wave w takes pages w, w+4, ...), each with
// a private online-softmax state, and merge the 4 states in LDS in wave order.
// The split launches (paged_decode_stream.h) keep the same 4 states per split
// (state s takes the split's pages start+s, start+s+4, ...) and merge them
// with the same arithmetic, so a row that fits in one split gives the same
// bits from the single-pass launch and from a split launch.
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
//     col n < G is query head kvh·G + n (the GQA group; with G > 16, head n of the
//     column group), the rest is zero padding.
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

// Query-head columns: one MFMA tile holds 16 heads, so a GQA group of G > 16
// heads is cut into ceil(G/16) column groups of at most 16 heads, each
// computed like a KV head of its own (the column groups of one KV head read the
// same K/V pages). For G <= 16 a KV head is one column group of G heads.
struct ColGroup {
  int kvh;    // KV head whose pages the column group reads
  int head0;  // first query head of the column group
  int cols;   // query heads in it (<= 16)
};
__device__ __forceinline__ int col_groups_per_kv(int G) { return (G + 15) >> 4; }
__device__ __forceinline__ ColGroup col_group(int G, int cg) {
  const int T = col_groups_per_kv(G);
  ColGroup c;
  c.kvh = cg / T;
  const int t = cg - c.kvh * T;
  c.head0 = c.kvh * G + 16 * t;
  c.cols = min(16, G - 16 * t);
  return c;
}

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
template <int D, bool NT = true>
__device__ __forceinline__ void gload(RowSlice<D>& r, const uint16_t* base, uint32_t off_elems) {
  const uint32_t off = off_elems * 2;
  if constexpr (NT) {
    if constexpr (D / 16 == 8) asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(r) : "v"(off), "s"(base));
    else asm volatile("global_load_dwordx2 %0, %1, %2 nt" : "=v"(r) : "v"(off), "s"(base));
  } else {
    if constexpr (D / 16 == 8) asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(r) : "v"(off), "s"(base));
    else asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(r) : "v"(off), "s"(base));
  }
}

template <int D, bool NT = true>
__device__ __forceinline__ void load_page(PageRegs<D>& r, const uint16_t* kbase, const uint16_t* vbase,
                                          const uint32_t (&off)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) gload<D, NT>(r.k[j], kbase, off[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) gload<D, NT>(r.v[j], vbase, off[j]);
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

// Sᵀ of one page: the D/32 MFMAs of K·Qᵀ in k-step order, from the K operand
// chunks kop[c] = K row n, dims 8(4c+g) .. +8 (lane n + 16g). Every page path
// (K through a transpose tile or straight from a staged page in LDS) forms
// the same operands and the same chain, so its scores have the same bits.
template <int D>
__device__ __forceinline__ f32x4_t page_scores(const uint4 (&kop)[D / 32], const uint4 (&qb)[D / 32]) {
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < D / 32; ++c) s = mfma_16x16x32(kop[c], qb[c], s);
  return s;
}

// The online softmax and PV product of one page, from its scores s (lane
// n + 16g holds S[head n][token 4g+i]) and its V rows v[j] = V row 4g+j, dims
// (D/16)·n .. +D/16, in three phases so that a wave with several independent
// states can interleave their pages (a dependent VALU operation waits about
// 36 clocks for its operand on gfx950, so one page alone is latency-bound):
//   softmax_phase: scores, running max and sum, P, and the PV operands;
//   rescale_phase: the accumulator rescale, skipped when every lane has
//                  alpha = 1 (x·1 == x) or a state that has seen no live
//                  token (its accumulators are +0, and +0·alpha = +0): both
//                  skips are exact, and the second saves a state's first page
//                  after every reset (each split's start) the rescale;
//   pv_phase:      the PV MFMAs.
// Tokens at or past tok_limit are masked: their scores become -inf and their
// V rows are replaced by zeros where they are used (unwritten slots may hold
// NaN, and 0·NaN would poison the PV product). The masking is branch-free so
// that loads in flight stay in flight.
template <int D>
struct PagePv {
  float alpha;
  bool fresh;          // the state had seen no live token (m = -inf): its accumulators are +0
  uint2 pb;            // P, bf16, B operand of the PV MFMAs
  uint2 va[D / 16];    // V^T operands (row = dim (D/16)·r + c, k = token 4g+i)
};

template <int D>
__device__ __forceinline__ void softmax_phase(WaveState<D>& st, PagePv<D>& ph, f32x4_t s,
                                              const RowSlice<D> (&v)[4], int tok0, int tok_limit,
                                              float scale_log2) {
  constexpr int VD = D / 16;
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
  ph.alpha = fast_exp2(st.m - m_ref);
  ph.fresh = st.m == kNegInf;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_ref);
  st.l = __builtin_fmaf(st.l, ph.alpha, (p[0] + p[1]) + (p[2] + p[3]));
  st.m = m_new;
  ph.pb.x = pack_bf16x2_hw(p[0], p[1]);
  ph.pb.y = pack_bf16x2_hw(p[2], p[3]);
  constexpr int VW = VD / 2;  // dwords per V row slice
  uint32_t vv[4][VW];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int x = 0; x < VW; ++x) vv[j][x] = live[j] ? v[j][x] : 0u;
  }
#pragma unroll
  for (int c = 0; c < VD; ++c) {
    ph.va[c].x = pick_halves(vv[0][c / 2], vv[1][c / 2], c & 1);
    ph.va[c].y = pick_halves(vv[2][c / 2], vv[3][c / 2], c & 1);
  }
}

template <int D>
__device__ __forceinline__ void rescale_phase(WaveState<D>& st, const PagePv<D>& ph) {
  if (__builtin_amdgcn_ballot_w64(ph.alpha != 1.f && !ph.fresh) != 0) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) st.acc[c] *= ph.alpha;
  }
}

template <int D>
__device__ __forceinline__ void pv_phase(WaveState<D>& st, const PagePv<D>& ph) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) st.acc[c] = mfma_16x16x16(ph.va[c], ph.pb, st.acc[c]);
}

template <int D>
__device__ __forceinline__ void page_softmax_pv(WaveState<D>& st, f32x4_t s, const RowSlice<D> (&v)[4],
                                                int tok0, int tok_limit, float scale_log2) {
  PagePv<D> ph;
  softmax_phase<D>(st, ph, s, v, tok0, tok_limit, scale_log2);
  rescale_phase<D>(st, ph);
  pv_phase<D>(st, ph);
}

// One page from registers (the work-group path): K passes through the wave's
// transpose tile into the MFMA layout.
template <int D>
__device__ __forceinline__ void process_page(WaveState<D>& st, const PageRegs<D>& r, const uint4 (&qb)[D / 32],
                                             unsigned char* tile, int n, int g,
                                             int tok0, int tok_limit, float scale_log2) {
  constexpr int VD = D / 16;
  constexpr int PITCH = 2 * D + 16;  // bytes; the pad keeps 16-row column reads conflict-free
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<RowSlice<D>*>(tile + (4 * g + j) * PITCH + 2 * VD * n) = r.k[j];
  asm volatile("" ::: "memory");
  uint4 kop[D / 32];
#pragma unroll
  for (int c = 0; c < D / 32; ++c) kop[c] = ld16(tile + n * PITCH + 16 * (4 * c + g));
  const f32x4_t s = page_scores<D>(kop, qb);
  asm volatile("" ::: "memory");
  page_softmax_pv<D>(st, s, r.v, tok0, tok_limit, scale_log2);
}

// Bytes of one wave's K transpose tile: 16 rows of D bf16 + 16 bytes of pad.
template <int D>
constexpr int kTileBytes = 16 * (2 * D + 16);

// The 4 wave states of a work-group as merge records in LDS, laid out for the
// reader: wave e merges element e of every lane's accumulator vectors, so
// lane L of wave e finds everything it needs in two blocks it reads with
// 16-byte loads and one wait:
//   [8L .. 8L+8):            m of states 0..3, then their row sums (over the
//                            four lane groups, the same in all four);
//   [512 + (64e + L)·R ..):  element e of accumulator vector c of state s at
//                            D/16·s + c (head n, dim D/16·(4g + e) + c;
//                            L = n + 16g), the row padded to R floats so that
//                            the 16-byte accesses of 16 lanes hit 64 banks.
template <int D>
constexpr int kMergeRowFloats = 4 * (D / 16) + 4;
template <int D>
constexpr int kMergeFloats = 64 * 8 + 4 * 64 * kMergeRowFloats<D>;

template <int D>
__device__ __forceinline__ void save_state(float* rec, const WaveState<D>& st, int s, int lane) {
  constexpr int VD = D / 16;
  rec[8 * lane + s] = st.m;
  rec[8 * lane + 4 + s] = sum_across_groups(st.l);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float* dst = rec + 512 + (64 * e + lane) * kMergeRowFloats<D> + VD * s;
#pragma unroll
    for (int c = 0; c < VD; c += 4)
      *reinterpret_cast<f32x4_t*>(dst + c) = f32x4_t{st.acc[c][e], st.acc[c + 1][e], st.acc[c + 2][e], st.acc[c + 3][e]};
  }
}

// Merge arithmetic of NS per-state results of one split, in state order:
// M = max of the states' maxima; L and A are fma chains in state order of the
// states' sums and accumulators weighted by 2^(m_s − M); o = A · (1 / L), or 0
// when no token was live (L = 0); lse = M + log2 L (−inf when L = 0). Every
// decode path merges a split's states with these functions (from LDS records
// in the work-group, from registers in the streaming wave), so a split's
// (o, lse) has the same bits whichever path computed it.
__device__ __forceinline__ float split_inv(float L) { return L > 0.f ? 1.f / L : 0.f; }
__device__ __forceinline__ float split_lse(float M, float L) { return L > 0.f ? M + __log2f(L) : kNegInf; }

// Merges the 4 wave states of the row (one split: the single-pass launch) in
// wave order for element e of every lane's accumulator vectors (records laid
// out by save_state), and writes those dims of the bf16 output rows of the G
// heads head0 .. head0 + G - 1 (one column group): lane (n, g) writes head n,
// dims VD·(4g + e) .. +VD-1.
template <int D>
__device__ __forceinline__ void merge_states(const DecodeArgs& a, const float* rec, int e, int G, int row,
                                             int head0, int lane) {
  constexpr int VD = D / 16;
  const int n = lane & 15;
  const int g = lane >> 4;
  const f32x4_t m4 = *reinterpret_cast<const f32x4_t*>(rec + 8 * lane);
  const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(rec + 8 * lane + 4);
  const float* row_e = rec + 512 + (64 * e + lane) * kMergeRowFloats<D>;
  f32x4_t av[VD];  // 4 states x VD elements, state-major
#pragma unroll
  for (int k = 0; k < VD; ++k) av[k] = *reinterpret_cast<const f32x4_t*>(row_e + 4 * k);
  float M = kNegInf;
#pragma unroll
  for (int s = 0; s < 4; ++s) M = fmaxf(M, m4[s]);
  float L = 0.f;
  float o[VD];
#pragma unroll
  for (int c = 0; c < VD; ++c) o[c] = 0.f;
  if (M != kNegInf) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float wgt = fast_exp2(m4[s] - M);
      L = __builtin_fmaf(l4[s], wgt, L);
#pragma unroll
      for (int c = 0; c < VD; ++c) o[c] = __builtin_fmaf(av[(VD * s + c) / 4][(VD * s + c) % 4], wgt, o[c]);
    }
  }
  const float inv = split_inv(L);
#pragma unroll
  for (int c = 0; c < VD; ++c) o[c] = L == 0.f ? 0.f : o[c] * inv;
  if (n < G) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.o_sb + (int64_t)(head0 + n) * a.o_sh +
                    VD * (4 * g + e);
    if constexpr (VD == 8) {
      uint4 pk;
      pk.x = pack_bf16x2_hw(o[0], o[1]);
      pk.y = pack_bf16x2_hw(o[2], o[3]);
      pk.z = pack_bf16x2_hw(o[4], o[5]);
      pk.w = pack_bf16x2_hw(o[6], o[7]);
      st16(dst, pk);
    } else {
      uint2 pk;
      pk.x = pack_bf16x2_hw(o[0], o[1]);
      pk.y = pack_bf16x2_hw(o[2], o[3]);
      st8(dst, pk);
    }
  }
}

// LDS bytes one decode work-group uses: NW K transpose tiles, then NW merge
// records.
template <int D, int NW>
constexpr size_t decode_lds_bytes() {
  static_assert(NW == 4, "the merge records hold four states");
  return (size_t)NW * kTileBytes<D> + (size_t)kMergeFloats<D> * sizeof(float);
}

// One single-pass decode work-group: (sequence, column group) = wg (a column
// group is a KV head when G <= 16), with NW waves and `smem` pointing at
// decode_lds_bytes<D, NW>() bytes of LDS. Wave w walks the row's pages w,
// w + NW, ... with PF pages in flight; the NW states are merged in wave order
// and the bf16 output rows are written.
// EAGER (PF = 1): page k+1 is requested as soon as page k has landed, before
// page k is computed (two register sets), instead of after; the page order, so
// the arithmetic, is the same either way.
template <int D, int NW, int PF, bool EAGER = false>
__device__ __forceinline__ void decode_work_group(const DecodeArgs& a, const int wg, float* smem) {
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;

  const int ncg = a.num_kv_heads * col_groups_per_kv(a.num_heads / a.num_kv_heads);
  const ColGroup cgp = col_group(a.num_heads / a.num_kv_heads, wg % ncg);
  const int G = cgp.cols;  // heads of this column group
  const int kvh = cgp.kvh;
  const int b = wg / ncg;

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

  // Qᵀ operand: lane (n + 16g), chunk c -> q[b][head0 + n][8(4c+g) .. +8).
  uint4 qb[KC];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)row * a.q_sb +
                           (int64_t)(cgp.head0 + n) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c) qb[c] = (n < G) ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }

  WaveState<D> st;
  st.m = kNegInf;
  st.l = 0.f;
#pragma unroll
  for (int c = 0; c < VD; ++c) st.acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t off[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) off[j] = (uint32_t)((4 * g + j) * a.c_st + VD * n);
  unsigned char* tile = reinterpret_cast<unsigned char*>(smem) + w * kTileBytes<D>;

  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  const int first = w;
  const int cnt = (n_blocks > first) ? (n_blocks - first + NW - 1) / NW : 0;
  // Lane k holds the table entry of this wave's page number base + k. The first
  // slice is requested together with seq_len and q (its index is clamped into
  // the row, so it does not wait for seq_len); entries past the row are unused.
  int ent = bt[min(first + NW * lane, a.max_blocks - 1)];
  for (int base = 0; base < cnt; base += 64) {
    const int here = min(64, cnt - base);
    if (base > 0) ent = bt[min(first + NW * (base + lane), a.max_blocks - 1)];
    const int slot_ent = min(max(ent, 0), a.num_pages - 1);
    auto phys = [&](int k) -> int64_t { return (int64_t)__builtin_amdgcn_readlane(slot_ent, k); };

    if constexpr (EAGER) {
      // One page in flight: page j+1 is requested as soon as page j has
      // landed (before page j is computed), and only while there is one: no
      // load is issued past the wave's last page, so the wave never waits at
      // its end for a page nobody computes. With at most one page outstanding
      // every wait is vmcnt(0).
      static_assert(PF == 1, "the eager walk keeps one page in flight");
      PageRegs<D> r[2];
      {
        const int64_t p = phys(0) * a.c_sb;
        load_page<D>(r[0], kc + p, vc + p, off);
      }
      for (int k = 0; k < here; k += 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (k + i < here) {
            wait_page<0, D>(r[i]);
            if (k + i + 1 < here) {
              const int64_t pn = phys(k + i + 1) * a.c_sb;
              load_page<D>(r[i ^ 1], kc + pn, vc + pn, off);
            }
            const int page = first + NW * (base + k + i);
            process_page<D>(st, r[i], qb, tile, n, g, page * 16 + 4 * g, seq_len, a.scale_log2);
          }
        }
      }
      // Every load issued above was waited for; this wait (immediate) keeps
      // that visible in the code's structure as well.
#pragma unroll
      for (int i = 0; i < 2; ++i) wait_page<0, D>(r[i]);
      continue;
    }
    // PF pages in flight per wave: page k+PF is requested as soon as page k has
    // been computed. Loads are issued unconditionally (page index clamped into
    // the wave's range) and the page count is padded to a multiple of PF with
    // fully masked pages, so every wait counts exactly PF-1 younger pages.
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
        const int page = first + NW * (base + k + i);
        const int limit = (k + i < here) ? seq_len : 0;
        process_page<D>(st, r[i], qb, tile, n, g, page * 16 + 4 * g, limit, a.scale_log2);
        const int64_t pn = phys(min(k + i + PF, here - 1)) * a.c_sb;
        load_page<D>(r[i], kc + pn, vc + pn, off);
      }
    }
    // Drain: the loads issued for pages past the end must land before their
    // registers are reused.
#pragma unroll
    for (int i = 0; i < PF; ++i) wait_page<0, D>(r[i]);
  }

  // Every wave saves its state (the merge records follow the NW K tiles);
  // then wave w merges element w of every lane's accumulator vectors and
  // writes those dims of the output rows.
  static_assert(NW == 4, "wave w merges element w of the 4-element accumulator vectors");
  float* merge = smem + NW * kTileBytes<D> / 4;
  save_state<D>(merge, st, w, lane);
  __syncthreads();
  merge_states<D>(a, merge, w, G, row, cgp.head0, lane);
}

}  // namespace bvllm
