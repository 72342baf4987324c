// Varlen paged prefill attention: causal GQA attention for a flattened batch of
// sequences whose keys/values (cached prefix + the step's new tokens) are read
// straight from the paged cache through the block table.
//
// Replaces paged_prefill_attn_kernel (babyvllm/kernels/paged_prefill.py:6-101).
//
// Work-group = (sequence, KV head, block of CB columns). The columns are the
// sequence's (query, head) pairs of the KV head's G query heads, numbered
// query-major (f = query·G + head), so every K/V tile is staged once per
// work-group and shared by the whole GQA group, and every MFMA column holds a
// pair whatever G is (a 16-column tile may span queries: the causal limit is
// per column). Each of the NW waves owns QT 16-column tiles; CB = NW·QT·16
// (with the key split KS = 2, below: pairs of waves share their tiles and each
// takes one half of every key tile; CB = NW/2·QT·16).
// Keys come in tiles of 64 (four 16-token pages), moved from the cache into LDS
// by direct global->LDS loads (no staging registers), rows XOR-swizzled instead
// of padded. K and V each have two LDS buffers; K runs one tile ahead of V.
// The products run on mfma 16x16x32 over halves of 32 keys:
//   Sᵀ[16 keys × 16 cols] = K · Qᵀ       (K operand from LDS)
//   Oᵀ[D × 16 cols]      += Vᵀ · Pᵀ      (Pᵀ from the Sᵀ registers, Vᵀ by LDS
//                                         transpose reads)
// software-pipelined by half: Sᵀ of the next half is computed while P of the
// current half is formed, so MFMA and VALU work of one wave overlap. P uses
// the running max as its reference; only when some P exceeds 2^8 (a score
// above the reference by more than 8 in log2 units) is the max raised and P
// formed again, so the max never delays P. The row sums come from an MFMA of P with
// an all-ones operand, next to the PV product.
// Keys at or past hi = min(seq_len, ctx + last query + 1) are masked, and their
// V rows are zeroed in LDS, so cache slots that were never written (possibly
// NaN) never reach a product.
//
// Sequences with a single query token (the decode rows of a mixed step) are
// instead computed by decode work-groups (paged_decode_wg.h) placed behind the
// prefill work-groups of the same launch: their waves split a row's pages,
// where a prefill work-group would walk them with one live wave.
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"
#include "paged_decode_wg.h"

#include <stdlib.h>

namespace bvllm {

// Blocks of CB columns (a sequence's q_len·G (query, head) pairs, numbered
// query-major) are numbered sequence by sequence, the blocks of a sequence last
// (most keys) first; a sequence with one query token has none when the decode
// work-groups compute it. Finds the sequence s and block qb of number r, or
// returns false if r is past the last block. Every wave computes the same
// wave-uniform answer (a scan of the per-sequence block counts).
__device__ __forceinline__ bool find_query_block(const PrefillArgs& a, int CB, int r, int& s_out, int& qb_out) {
  const int G = a.num_heads / a.num_kv_heads;
  constexpr int kChunk = 4;  // 64-sequence slices whose counts are loaded together
  const int lane = lane_id();
  int before = 0;
  for (int s0 = 0; s0 < a.num_seqs; s0 += 64 * kChunk) {
    int nb[kChunk];
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int s = s0 + 64 * c + lane;
      nb[c] = 0;
      if (s < a.num_seqs) {
        const int ql = a.query_start_loc[s + 1] - a.query_start_loc[s];
        nb[c] = (ql == 1 && a.single_query_seqs != 0) ? 0 : (ql * G + CB - 1) / CB;
      }
    }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      int inc = nb[c];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(inc, d, 64);
        if (lane >= d) inc += t;
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(before + inc > r);
      if (hit != 0) {
        const int l = (int)__builtin_ctzll(hit);
        const int nb_l = __shfl(nb[c], l, 64);
        const int first = before + __shfl(inc, l, 64) - nb_l;
        s_out = uniform(s0 + 64 * c + l);
        qb_out = uniform(nb_l - 1 - (r - first));
        return true;
      }
      before += __shfl(inc, 63, 64);
    }
  }
  return false;
}

// Waves and pages in flight of the decode work-groups of a mixed step: one page
// per wave, the next requested as soon as it has landed and none past the
// wave's last page (1 x 512 + 63 decodes: 28.4 us, against 29.9 with two pages
// requested after each page is computed).
constexpr int kDecodeWaves = 4;
constexpr int kDecodeDepth = 1;

// MB: groups of several blocks per work-group, launched only when every
// sequence's keys fit two 64-key tiles (the kernel has no streaming path then).
// KS: key split inside the work-group. KS = 1: each wave owns QT column tiles
// and walks every key. KS = 2: the waves form NW/2 column groups of QT tiles,
// and the two waves of a group take the two 32-key halves of every 64-key tile
// (twice the columns per LDS read of K and V and per staged tile, for the same
// waves); their partial states merge through LDS at the end.
template <int D, int NW, int QT, bool MB, int KS>
__global__ __launch_bounds__(NW * 64, 2) void paged_prefill_kernel(PrefillArgs a, int n_blocks_bound, int dense_qb,
                                                                  int xcd_group, int per_xcd, DecodeArgs dec,
                                                                  int n_dec_wgs, int bpw) {
  constexpr int KT = 64;
  constexpr int RB = 2 * D;   // bytes of one key row of K or V (no padding)
  constexpr int TB = 64 * RB;  // bytes of one 64-key K or V tile
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int CPR = D / 8;
  constexpr int CHUNKS = KT * CPR;
  constexpr int PER_T = CHUNKS / (NW * 64);
  static_assert(PER_T * NW * 64 == CHUNKS, "tile chunks must divide evenly over the work-group");
  static_assert(KT == 64, "a key tile spans four 16-token pages");

  // K tiles in buffers 0 and 1, V tiles in buffers 2 and 3.
  __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * TB];
  static_assert(NW == kDecodeWaves, "decode work-groups run with the prefill work-group size");
  static_assert(decode_lds_bytes<D, kDecodeWaves>() <= sizeof(lds), "decode work-group LDS");

  // The last n_dec_wgs work-groups are decode work-groups, one per (sequence,
  // KV head); those past the batch have nothing to do. They come after the
  // prefill work-groups so that the prefill ones, dispatched first, get their
  // first tiles' loads in ahead of the decode work-groups' page stream, which
  // otherwise fills each CU's memory queue in front of them (mixed step
  // 1 x 512 + 63 decodes: 34.6 -> 29.5 us).
  const int n_pre_wgs = (int)gridDim.x - n_dec_wgs;
  if ((int)blockIdx.x >= n_pre_wgs) {
    const int dw = (int)blockIdx.x - n_pre_wgs;
    if (dw < dec.batch * dec.num_kv_heads * col_groups_per_kv(dec.num_heads / dec.num_kv_heads))
      decode_work_group<D, kDecodeWaves, kDecodeDepth, true>(dec, dw, reinterpret_cast<float*>(lds));
    return;
  }

  const int G = a.num_heads / a.num_kv_heads;
  static_assert(KS == 1 || (KS == 2 && !MB && NW % 2 == 0), "key split: two halves, streaming path only");
  constexpr int CB = NW / KS * QT * 16;  // columns of a work-group's block

  // Work-groups are dispatched round-robin over the 8 XCDs (XCD = id mod 8).
  // xcd_group == -1 (many (sequence, KV head) pairs, dense numbering): each XCD
  // takes a contiguous range of (sequence, KV head, block), so the blocks that
  // share a prefix share an L2 and every XCD gets many whole pairs.
  // xcd_group = 8 / Hkv > 0 (few pairs, or a mixed step): KV head h is served
  // by XCDs h·xcd_group .. +xcd_group-1, which deal its column blocks out in
  // boustrophedon order (0 1 | 1 0 | 0 1 ...): each L2 holds one KV head's
  // keys, and the heavy-to-light run of a sequence's blocks spreads evenly.
  const int id = blockIdx.x;
  // The arguments that address the metadata and table loads below, read
  // with the mapping's own: otherwise their wait splits those loads' round trip.
  asm volatile("" ::"s"(a.block_tables), "s"(a.bt_stride), "s"(a.max_blocks), "s"(a.query_start_loc),
               "s"(a.seq_lens), "s"(a.context_lens), "s"(a.q), "s"(a.q_st), "s"(a.q_sh), "s"(a.k_cache),
               "s"(a.v_cache), "s"(a.c_st), "s"(a.c_sh), "s"(a.c_sb), "s"(a.num_pages));
  int kvh, r;
  if (xcd_group < 0) {
    const int L = (id & 7) * per_xcd + (id >> 3);
    if (L >= n_blocks_bound * a.num_kv_heads) return;
    const int sk = L / dense_qb;
    kvh = sk % a.num_kv_heads;
    r = (sk / a.num_kv_heads) * dense_qb + (L - sk * dense_qb);
  } else if (xcd_group > 0) {
    const int x = id & 7;
    const int j = id >> 3;
    const int off = x % xcd_group;
    kvh = x / xcd_group;
    r = xcd_group * j + ((j & 1) ? xcd_group - 1 - off : off);
  } else {
    kvh = id % a.num_kv_heads;
    r = id / a.num_kv_heads;
  }
  if (r >= n_blocks_bound) return;
  int s, qb;
  if (dense_qb > 0) {
    // Dense numbering: every sequence owns dense_qb block numbers.
    s = r / dense_qb;
    qb = dense_qb - 1 - (r - s * dense_qb);
  } else if (!find_query_block(a, CB * (MB ? bpw : 1), r, s, qb)) {
    return;
  }

  // The sequence's metadata and the page numbers of its first two 64-key
  // tiles, as scalar loads (constant address space) issued together and
  // waited for once, above the returns below (a work-group that returns leaves
  // the entries unused): one round trip. A later tile's entries are fetched a
  // half step before their use. page_fetch issues the loads of tile kt's four
  // entries (entries past the row's last are clamped to it: only the last
  // tiles reach there); page_finish waits for them and forms byte offsets.
  typedef const int32_t __attribute__((address_space(4)))* ConstI32;
  int q_start = ((ConstI32)a.query_start_loc)[s];
  int q_end = ((ConstI32)a.query_start_loc)[s + 1];
  int seq_len = ((ConstI32)a.seq_lens)[s];
  int ctx = ((ConstI32)a.context_lens)[s];
  constexpr int PAGES_PER_TILE = KT / 16;
  static_assert(PAGES_PER_TILE == 4, "page_finish consumes four entries");
  const ConstI32 bts = (ConstI32)(a.block_tables + (int64_t)s * a.bt_stride);
  const uint32_t page_bytes = (uint32_t)a.c_sb * 2u;  // c_sb < 2^31, checked on the host
  // (No branch between the fast and the clamped form: the waits that close
  // each side of one would split the loads' round trip.)
  // KS = 2 forms the entry addresses as 32-bit byte offsets (a scalar load
  // with a register offset: three scalar instructions per entry instead of
  // six) and clamps entries as unsigned (a negative entry maps to the last
  // page instead of page 0; either is an in-bounds load of a tile that no
  // result reads): 8 x (1024+128) 30.9 -> 30.35 us. The streaming walk keeps
  // the signed form (1 x (2048+4096): 213.4 against 219.6 us with this one,
  // from the compiler's schedule of the rest of the step). Entries past
  // 2^28 are never needed (seq_len < 2^31 is at most 2^27 pages), which
  // keeps the byte offsets inside 32 bits.
  typedef const char __attribute__((address_space(4)))* ConstBytes;
  const uint32_t bt_last = (uint32_t)min(a.max_blocks - 1, 1 << 28) * 4u;
  const uint32_t page_last = (uint32_t)(a.num_pages - 1);
  auto page_fetch = [&](int kt, int (&raw)[PAGES_PER_TILE]) __attribute__((always_inline)) {
    if constexpr (KS == 2) {
      const uint32_t o0 = (uint32_t)kt * (4u * PAGES_PER_TILE);
#pragma unroll
      for (int pg = 0; pg < PAGES_PER_TILE; ++pg)
        raw[pg] = *(ConstI32)((ConstBytes)bts + (uint64_t)min(o0 + 4u * pg, bt_last));
    } else {
      const int i0 = kt * PAGES_PER_TILE;
#pragma unroll
      for (int pg = 0; pg < PAGES_PER_TILE; ++pg) raw[pg] = bts[min(i0 + pg, a.max_blocks - 1)];
    }
  };
  auto page_finish = [&](int (&raw)[PAGES_PER_TILE], int64_t (&po)[PAGES_PER_TILE]) __attribute__((always_inline)) {
    asm volatile("" : "+s"(raw[0]), "+s"(raw[1]), "+s"(raw[2]), "+s"(raw[3]));
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) {
      if constexpr (KS == 2) po[pg] = (int64_t)((uint64_t)min((uint32_t)raw[pg], page_last) * page_bytes);
      else po[pg] = (int64_t)((uint64_t)(uint32_t)min(max(raw[pg], 0), a.num_pages - 1) * page_bytes);
    }
  };
  int64_t po_v[PAGES_PER_TILE], po_k[PAGES_PER_TILE], po_n[PAGES_PER_TILE];
  {
    int raw0[PAGES_PER_TILE], raw1[PAGES_PER_TILE], raw2[PAGES_PER_TILE];
    page_fetch(0, raw0);
    page_fetch(1, raw1);
    if constexpr (KS == 2) page_fetch(2, raw2);
    asm volatile("" : "+s"(q_start), "+s"(q_end), "+s"(seq_len), "+s"(ctx));
    page_finish(raw0, po_v);
    page_finish(raw1, po_k);
    if constexpr (KS == 2) page_finish(raw2, po_n);
  }
  const int q_len = q_end - q_start;
  const int n_cols = q_len * G;
  // qb numbers groups of nbpw blocks of CB columns (one block unless MB); the
  // work-group computes the group's blocks one after another, the last (most
  // keys) first. Every block of an MB group reads the same (at most two)
  // tiles: they are staged once, and the later blocks only load their Q.
  const int nbpw = MB ? bpw : 1;
  if (qb * nbpw * CB >= n_cols) return;
  if (q_len == 1 && a.single_query_seqs != 0) return;  // on the decode work-groups
  const int b_first = qb * nbpw;
  const int b_last = min(b_first + nbpw, (n_cols + CB - 1) / CB) - 1;

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;
  const int w = wave_id();
  const int cw = w % (NW / KS);  // the wave's column group
  const int kh = w / (NW / KS);  // KS = 2: the 32-key half of every tile the wave takes

  bool kv_staged = false;
  int blk = b_last;
  do {  // blocks of the group (a single pass unless MB)
  const int q_last = (min(n_cols, (blk + 1) * CB) - 1) / G;
  // (MB: the host checked that no sequence has more than two tiles' pages;
  // the clamp keeps an inconsistent seq_lens inside the staged tiles.)
  const int hi = min(min(seq_len, ctx + q_last + 1), MB ? 2 * KT : 0x7fffffff);
  const int n_tiles = hi > 0 ? (hi + KT - 1) / KT : 0;

  // The wave's columns: f = wave_f0 + 16·ct + n of the block's flat
  // (query, head) numbering, query f / G and head f mod G.
  const int wave_f0 = blk * CB + cw * QT * 16;
  const int wave_q0 = wave_f0 / G;  // first query index of this wave
  const bool wave_live = wave_f0 < n_cols;
  const int wave_hi = ctx + min(q_len - 1, (wave_f0 + QT * 16 - 1) / G);  // last visible key position

  int qi[QT], hl[QT];
  int qpos[QT];
  bool valid[QT];
  uint4 qreg[QT][KC];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    const int f = wave_f0 + 16 * ct + n;
    qi[ct] = f / G;
    hl[ct] = f - qi[ct] * G;
    valid[ct] = f < n_cols;
    qpos[ct] = valid[ct] ? ctx + qi[ct] : 0x7fffffff;
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)(q_start + qi[ct]) * a.q_st +
                           (int64_t)(kvh * G + hl[ct]) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[ct][c] = valid[ct] ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }


  // lsum[ct]: the running row sums of P, accumulated by an MFMA of an all-ones
  // operand with the same bf16 P that multiplies V (every row of the result
  // holds the column sums), so numerator and denominator sum the same values.
  float m[QT];
  f32x4_t acc[QT][VD], lsum[QT];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    m[ct] = kNegInf;
    lsum[ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < VD; ++c) acc[ct][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint4 ones_bf16 = make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);

  const unsigned char* kc = reinterpret_cast<const unsigned char*>(a.k_cache) + (int64_t)kvh * a.c_sh * 2;
  const unsigned char* vc = reinterpret_cast<const unsigned char*>(a.v_cache) + (int64_t)kvh * a.c_sh * 2;

  // Staging: direct global -> LDS loads (global_load_lds_dwordx4). One load
  // of a wave moves 64 chunks of 16 B into 1 KB of LDS, lane i to byte 16·i:
  // block e = r·NW + w (r < PER_T) of a tile holds key rows RPB·e .. +RPB-1
  // (RPB = 1024 / RB). Rows are unpadded; instead each row's 16-byte chunks are
  // XOR-swizzled by the row's position in its page (rt = key mod 16):
  //   K chunk c sits at c ^ (rt mod CPR)            (16 rows read per 16 lanes)
  //   V chunk c sits at c ^ 2·(rt mod CPR/2)        (pairs stay adjacent for the
  //                                                   32-byte transpose reads)
  // so both read patterns are bank-conflict-free. Lane i loads the global
  // chunk that belongs at its LDS position. Tiles start on page boundaries and
  // NW·RPB is a multiple of 16, so rt and both source offsets are the same on
  // every tile and every r; the page of block e is r·PG_STEP + (wave offset).
  constexpr int RPB = 1024 / RB;
  constexpr int PG_STEP = NW * 64 / (2 * D);
  static_assert(RPB * PER_T * NW == KT, "a tile is PER_T loads per wave");
  static_assert((NW * RPB) % 16 == 0, "row-in-page of a lane is the same for every r");
  static_assert(PG_STEP * 2 * D == NW * 64 && PG_STEP * PER_T == PAGES_PER_TILE, "staging page layout");
  static_assert(PG_STEP == 1 || PG_STEP == 2, "a wave's block of one r lies in page r·PG_STEP + (0 or 1)");
  const int pg_wave = uniform((int)(threadIdx.x / (2 * D)));  // always 0 when PG_STEP == 1
  const int st_rt = (w * RPB + lane / CPR) & 15;             // the lane's row within its page
  const int st_pos = lane % CPR;                              // the lane's chunk position in the row
  const uint32_t st_off_k = (uint32_t)(((int64_t)st_rt * a.c_st + (st_pos ^ (st_rt & (CPR - 1))) * 8) * 2);
  const uint32_t st_off_v =
      (uint32_t)(((int64_t)st_rt * a.c_st + (st_pos ^ (2 * (st_rt & (CPR / 2 - 1)))) * 8) * 2);
  const uint32_t lds_base = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) unsigned char*)lds);
  const uint32_t lds_wave = lds_base + (uint32_t)w * 1024u;


  // The loads are inline asm, invisible to the compiler's wait insertion
  // (which would otherwise wait for them before every LDS read); each wave
  // waits for its own loads (vmcnt) before the barrier that publishes a tile.
  // M0 holds the wave's LDS destination.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  auto dma = [&](const unsigned char* gbase, uint32_t off, uint32_t lds_addr) __attribute__((always_inline)) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds_addr), "v"(off), "s"(gbase)
                 : "memory", "m0");
  };
#pragma clang diagnostic pop
  auto page_of = [&](const int64_t (&po)[PAGES_PER_TILE], int r) __attribute__((always_inline)) -> int64_t  {
    if constexpr (PG_STEP == 1) return po[r];
    else return pg_wave ? po[PG_STEP * r + 1] : po[PG_STEP * r];
  };
  auto stage_k = [&](const int64_t (&po)[PAGES_PER_TILE], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) dma(kc + page_of(po, r), st_off_k, lds_wave + buf * TB + r * NW * 1024);
  };
  auto stage_v = [&](const int64_t (&po)[PAGES_PER_TILE], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) dma(vc + page_of(po, r), st_off_v, lds_wave + (2 + buf) * TB + r * NW * 1024);
  };
  // After the wave's loads landed: V rows of tile kt at or past hi become
  // zeros (unwritten slots may hold NaN, and 0·NaN would poison the PV
  // product). K rows there only reach scores that the mask replaces by -inf.
  auto zero_v_tail = [&](int kt, int buf) __attribute__((always_inline)) {
    if (kt * KT + KT > hi) {  // uniform
#pragma unroll
      for (int r = 0; r < PER_T; ++r) {
        const int row = (r * NW + w) * RPB + lane / CPR;
        if (kt * KT + row >= hi)
          *reinterpret_cast<u32x4_t*>(lds + (2 + buf) * TB + (r * NW + w) * 1024 + lane * 16) =
              u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  };
  auto wait_loads = [&]() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };

  // Last visible key of each column (its query position, at most hi - 1):
  // on tiles that reach past a column's diagonal or past hi, key pos is masked
  // for the column iff pos > lim.
  int lim[QT];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) lim[ct] = min(qpos[ct], hi - 1);
  // 32-key halves of tiles this wave computes: up to its last visible key
  // (wave_hi) and below hi.
  const int wave_halves = wave_live ? min((hi + 31) / 32, wave_hi / 32 + 1) : 0;
  // KS = 2: tiles whose half kh holds a key this wave's columns see.
  const int wave_last_key = min(wave_hi, hi - 1);
  const int wave_tiles = (KS == 2 && wave_live && wave_last_key >= 32 * kh) ? (wave_last_key - 32 * kh) / 64 + 1 : 0;

  // ---- products and softmax, per 32-key half of a 64-key tile ----
  // Sᵀ of keys 32h .. 32h+31 of the tile in K buffer kbuf, for the wave's QT
  // column tiles: S[ct][t'] holds keys 32h + 16t' + 4g + i (lane n = column).
  uint32_t k_off[KC];  // row n (its row in page is n), chunk 4c + g
#pragma unroll
  for (int c = 0; c < KC; ++c) k_off[c] = (uint32_t)(n * RB + 16 * ((4 * c + g) ^ (n & (CPR - 1))));
  auto qk = [&](f32x4_t (&S)[QT][2], int kbuf, const int h) __attribute__((always_inline)) {
    const unsigned char* K = lds + kbuf * TB + 32 * h * RB;
#pragma unroll
    for (int ct = 0; ct < QT; ++ct)
#pragma unroll
      for (int t = 0; t < 2; ++t) S[ct][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const uint4 ka = ld16(K + 16 * t * RB + k_off[c]);
#pragma unroll
        for (int ct = 0; ct < QT; ++ct) S[ct][t] = mfma_16x16x32(ka, qreg[ct][c], S[ct][t]);
      }
    }
  };
  // Causal / hi mask of a half whose first key is k0 (absolute position):
  // key k0 + 16t + 4g + i is masked iff 16t + i > lim - k0 - 4g.
  auto mask = [&](f32x4_t (&S)[QT][2], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) {
      const int rel = lim[ct] - k0 - 4 * g;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (16 * t + i > rel) S[ct][t][i] = kNegInf;
    }
  };
  // Some key of the half at k0 may be invisible to some column of the wave.
  auto needs_mask = [&](int k0) { return (k0 + 31 > ctx + wave_q0) || (k0 + 32 > hi); };
  // The scores' max of each column over a half, in log2 units (the scale is
  // > 0, so it commutes with the max): a chain of three-input maxima, then
  // across the four lane groups.
  auto half_max1 = [&](const f32x4_t (&S)[QT][2], const int ct) __attribute__((always_inline)) -> float {
    float mx = fmax_prop(fmax_prop(S[ct][0][0], S[ct][0][1]), S[ct][0][2]);
    mx = fmax_prop(fmax_prop(mx, S[ct][0][3]), S[ct][1][0]);
    mx = fmax_prop(fmax_prop(mx, S[ct][1][1]), S[ct][1][2]);
    mx = fmax_prop(mx, S[ct][1][3]);
    return max_across_groups(mx) * a.scale_log2;
  };
  auto half_max = [&](const f32x4_t (&S)[QT][2], float (&mt)[QT]) __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) mt[ct] = half_max1(S, ct);
  };
  // P = 2^(s·scale − m), packed to bf16 as the B operand of the PV product
  // over the half's 32 keys.
  float pmax[QT];  // the lane's largest P of the half, per column tile
  auto softmax_p1 = [&](const f32x4_t (&S)[QT][2], uint4 (&pb)[QT], const int ct) __attribute__((always_inline)) {
    float p[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) p[t][i] = fast_exp2(__builtin_fmaf(S[ct][t][i], a.scale_log2, -m[ct]));
    float px = fmax_prop(fmax_prop(p[0][0], p[0][1]), p[0][2]);
    px = fmax_prop(fmax_prop(px, p[0][3]), p[1][0]);
    px = fmax_prop(fmax_prop(px, p[1][1]), p[1][2]);
    pmax[ct] = fmax_prop(px, p[1][3]);
    pb[ct].x = pack_bf16x2_hw(p[0][0], p[0][1]);
    pb[ct].y = pack_bf16x2_hw(p[0][2], p[0][3]);
    pb[ct].z = pack_bf16x2_hw(p[1][0], p[1][1]);
    pb[ct].w = pack_bf16x2_hw(p[1][2], p[1][3]);
  };
  auto softmax_p = [&](const f32x4_t (&S)[QT][2], uint4 (&pb)[QT]) __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) softmax_p1(S, pb, ct);
  };
  // The running max m is the reference of P = 2^(s·scale − m). It is raised
  // only when some column's new max exceeds it by more than 8 (a factor 256;
  // P stays far inside fp32 and bf16 range, and the final division by the
  // row sum removes the common factor): then acc and the row sums are
  // rescaled by 2^(m_old − m_new) and P is formed again. That happens exactly
  // when some P of the column exceeds 2^8, so each lane tests the largest of
  // its own P (formed anyway), a ballot joins the lanes, and only on this rare
  // path is the column max itself formed: P never waits for a max, and the
  // common path has no cross-lane reduction.
  auto raise_max = [&](const f32x4_t (&S)[QT][2], uint4 (&pb)[QT]) __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) {
      if (__builtin_amdgcn_ballot_w64(!(pmax[ct] <= 256.0f)) != 0) {
        const float m_new = fmax_prop(m[ct], half_max1(S, ct));
        const float alpha = fast_exp2(m[ct] - m_new);
        m[ct] = m_new;
#pragma unroll
        for (int c = 0; c < VD; ++c) acc[ct][c] *= alpha;
        lsum[ct] *= alpha;
        softmax_p1(S, pb, ct);
      }
    }
  };
  // Lane n of group g addresses row 32h + 4g + n/4 (and +16), bytes
  // 32c + 8(n mod 4), i.e. chunk 2c + (n mod 4)/2, stored at that chunk ^
  // 2·(row mod CPR/2); 32h and 16 do not change the row's swizzle, so the
  // lane's offset for dim block c is fixed and h, +16 and the buffer enter as
  // constants.
  uint32_t v_off[VD];
  {
    const int tr_row = 4 * g + (n >> 2);
    const int sw = 2 * (tr_row & (CPR / 2 - 1));
#pragma unroll
    for (int c = 0; c < VD; ++c)
      v_off[c] = (uint32_t)(tr_row * RB + 16 * ((2 * c + ((n & 3) >> 1)) ^ sw) + 8 * (n & 1));
  }
  auto pv = [&](const uint4 (&pb)[QT], int vbuf, const int h) __attribute__((always_inline)) {
    const unsigned char* V = lds + (2 + vbuf) * TB + 32 * h * RB;
#pragma unroll
    for (int c = 0; c < VD; ++c) {
      const uint2 lo = ld_tr16(reinterpret_cast<const uint16_t*>(V + v_off[c]));
      const uint2 hi2 = ld_tr16(reinterpret_cast<const uint16_t*>(V + 16 * RB + v_off[c]));
      const uint4 va = make_uint4(lo.x, lo.y, hi2.x, hi2.y);
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) acc[ct][c] = mfma_16x16x32(va, pb[ct], acc[ct][c]);
    }
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) lsum[ct] = mfma_16x16x32(ones_bf16, pb[ct], lsum[ct]);
    // Schedule: the transpose reads run four dim blocks ahead of the MFMAs
    // that use them (8 reads, then per block its MFMAs and the next block's
    // two reads). Left to itself the compiler issued them two blocks ahead in
    // bursts, and every other block's MFMAs waited on LDS latency
    // (1 x (2048+4096): 222.9 -> 216.5 us; two blocks ahead 220.3, six 216.5,
    // all reads first 218.6; 64 x 128: 35.9 -> 35.2 us).
    constexpr int kAhead = VD < 4 ? VD : 4;
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kAhead, 0);  // DS reads
#pragma unroll
    for (int c = 0; c < VD - kAhead; ++c) {
      __builtin_amdgcn_sched_group_barrier(0x008, QT, 0);  // MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, (kAhead + 1) * QT, 0);
  };
  // Key split: the V operands of the wave's half (every dim block) are read
  // from LDS at the start of the tile step, before the next tile's QKᵀ, and a
  // scheduling barrier keeps them there: they depend only on the staged tile,
  // so their LDS round trips pass under the QKᵀ MFMAs and the softmax instead
  // of stalling the PV MFMAs group by group (as `pv`, whose reads the compiler
  // interleaves with its MFMAs through a few registers). 8 x (1024+128):
  // 30.8-31.1 -> 30.2-30.7 us; on the other paths the extra 32 live registers
  // cost more than they save (1 x (2048+4096): 225.5 -> 226.5 us).
  auto pv_load = [&](uint4 (&vop)[VD], int vbuf, const int h) __attribute__((always_inline)) {
    const unsigned char* V = lds + (2 + vbuf) * TB + 32 * h * RB;
#pragma unroll
    for (int c = 0; c < VD; ++c) {
      const uint2 lo = ld_tr16(reinterpret_cast<const uint16_t*>(V + v_off[c]));
      const uint2 hi2 = ld_tr16(reinterpret_cast<const uint16_t*>(V + 16 * RB + v_off[c]));
      vop[c] = make_uint4(lo.x, lo.y, hi2.x, hi2.y);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto pv_mma = [&](const uint4 (&pb)[QT], const uint4 (&vop)[VD]) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < VD; ++c)
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) acc[ct][c] = mfma_16x16x32(vop[c], pb[ct], acc[ct][c]);
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) lsum[ct] = mfma_16x16x32(ones_bf16, pb[ct], lsum[ct]);
  };

  // ---- pipeline over 32-key halves ----
  // Half x = 2j + h is keys 32x .. 32x+31 (tile j, half h). Half step x
  // computes Sᵀ(x+1) while forming P(x) from Sᵀ(x), rescales acc, masks
  // Sᵀ(x+1) if needed, then accumulates PV(x) while taking the max of Sᵀ(x+1).
  // Buffers: K(j) in K buffer j&1, V(j) in V buffer j&1.
  // A work-group with at most two tiles (short) loads all of them in the
  // prologue and then runs its halves with no loads, waits or barriers.
  // Otherwise the prologue loads K(0), V(0), K(1), and per tile j:
  //   start:  loads of V(j+1) into V buffer (j+1)&1 (V(j-1) is consumed);
  //   half 0: reads K(j) (its second half) and V(j);
  //   mid:    waits for K(j+1) (loaded since the previous mid), barrier —
  //           K(j+1) is published and K(j) is consumed everywhere — then
  //           loads K(j+2) into K buffer j&1;
  //   half 1: reads K(j+1) (its first half) and V(j);
  //   end:    waits for V(j+1), clears its rows past hi, barrier.
  // Loads are waited for in issue order (vmcnt), one tile step after issue;
  // the last steps load tiles past n_tiles (clamped table entries, in bounds)
  // that are never read, so the steady state has no branches around loads.
  // KS = 2 (a wave takes half kh of every tile): the prologue loads K(0),
  // V(0), K(1) and computes Sᵀ(0); step j then loads V(j+1) and K(j+2) (their
  // buffers' previous tiles were consumed in step j-1), computes Sᵀ(j+1) from
  // K(j+1) while forming P(j), accumulates PV(j), waits for its loads, clears
  // V(j+1)'s rows past hi and ends with the one barrier of the step. The
  // page numbers of tile j+3 are fetched under step j's products.
  const bool short_wg = KS == 1 && (MB || n_tiles <= 2);
  f32x4_t S0[QT][2], S1[QT][2];
  if (n_tiles > 0 && !(kv_staged && short_wg)) {
    stage_k(po_v, 0);
    stage_v(po_v, 0);
    if (n_tiles > 1 || !short_wg) stage_k(po_k, 1);
    if (short_wg && n_tiles == 2) stage_v(po_k, 1);
    wait_loads();
    zero_v_tail(0, 0);
    if (short_wg && n_tiles == 2) zero_v_tail(1, 1);
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) {
      po_v[pg] = po_k[pg];
      if constexpr (KS == 2) po_k[pg] = po_n[pg];
    }
  }
  kv_staged = short_wg;
  // The Q loads complete here, once, after the first tiles' table fetch and
  // loads were issued behind them: otherwise they look pending at the key
  // loop's header and the compiler drains every load there on each iteration.
#pragma unroll
  for (int ct = 0; ct < QT; ++ct)
#pragma unroll
    for (int c = 0; c < KC; ++c) asm volatile("" ::"v"(qreg[ct][c].x), "v"(qreg[ct][c].y), "v"(qreg[ct][c].z), "v"(qreg[ct][c].w));
  __syncthreads();
  if (KS == 1 ? wave_halves > 0 : wave_tiles > 0) {
    qk(S0, 0, KS == 2 ? kh : 0);
    if (needs_mask(32 * kh)) mask(S0, 32 * kh);
    // The first half's max is the first reference; a column with no visible
    // key yet takes 0 (its P is then 0, and a later max above 8 raises it).
    float mt[QT];
    half_max(S0, mt);
#pragma unroll
    for (int ct = 0; ct < QT; ++ct) m[ct] = mt[ct] == kNegInf ? 0.f : mt[ct];
  }
  // KS = 2: step 0 loads K(2) into K(0)'s buffer, which every wave has just
  // read for Sᵀ(0).
  if constexpr (KS == 2) __syncthreads();

  // Half step x (= 2j + h) on S(x) in Sc, producing S(x+1) in Sn.
  auto half_step = [&](const int x, f32x4_t (&Sc)[QT][2], f32x4_t (&Sn)[QT][2], const int kbuf_next,
                       const int h_next, const int vbuf, const int h, const bool next = true)
                       __attribute__((always_inline)) {
    // One code path for every computed half of the streaming walk: its last
    // half also forms Sᵀ(x+1) (in-bounds LDS reads of a buffer it never
    // uses), so that the accumulators have a single definition per step. The
    // short path passes next = false for a wave's last half, which skips that
    // product (64 x 128: 36.0 -> 35.6 us).
    uint4 pb[QT];
    if (x < wave_halves) {
      __builtin_amdgcn_s_setprio(1);
      if (next) qk(Sn, kbuf_next, h_next);
      softmax_p(Sc, pb);
      if constexpr (KS == 1 && !MB) {
        // Schedule: the K reads, then each QKᵀ MFMA followed by one VALU
        // instruction of P (1 x (2048+4096): 218.6 -> 214.9 us; two VALU per
        // MFMA 215.4, three 230.3, the K reads spread between the MFMAs 230.2;
        // the key-split step gains nothing measurable from the same groups).
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * KC, 0);  // DS reads
#pragma unroll
        for (int i = 0; i < 2 * KC * QT; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
        }
      }
      // P is formed here, under the QKᵀ MFMAs and beside the max, not sunk
      // past the branches below.
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) asm volatile("" ::"v"(pb[ct].x), "v"(pb[ct].y), "v"(pb[ct].z), "v"(pb[ct].w));
      __builtin_amdgcn_s_setprio(0);
      raise_max(Sc, pb);
      if (next && needs_mask(32 * (x + 1))) mask(Sn, 32 * (x + 1));
      __builtin_amdgcn_s_setprio(1);
      pv(pb, vbuf, h);
      __builtin_amdgcn_s_setprio(0);
    }
  };
  auto wait_older_loads = [&]() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_T) : "memory"); };
  // po_v holds the pages of tile j+1 (staged for K(j+1) at the previous mid
  // step or in the prologue) when step j starts.
  auto tile_step = [&](const int j, const int b) __attribute__((always_inline)) {  // b = j & 1
    int raw[PAGES_PER_TILE];
    page_fetch(j + 2, raw);
    stage_v(po_v, b ^ 1);
    half_step(2 * j, S0, S1, b, 1, b, 0);
    wait_older_loads();  // K(j+1)
    __syncthreads();
    page_finish(raw, po_k);
    stage_k(po_k, b);
    half_step(2 * j + 1, S1, S0, b ^ 1, 0, b, 1);
    wait_older_loads();  // V(j+1)
    zero_v_tail(j + 1, b ^ 1);
    __syncthreads();
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) po_v[pg] = po_k[pg];
  };
  // KS = 2: tile step j (b = j & 1) on Sᵀ(j) in Sc, producing Sᵀ(j+1) in Sn.
  auto split_step = [&](const int j, const int b, f32x4_t (&Sc)[QT][2], f32x4_t (&Sn)[QT][2])
                        __attribute__((always_inline)) {
    stage_v(po_v, b ^ 1);  // V(j+1)
    stage_k(po_k, b);      // K(j+2)
    int raw[PAGES_PER_TILE];
    page_fetch(j + 3, raw);
    if (j < wave_tiles) {
      uint4 pb[QT];
      uint4 vop[VD];
      pv_load(vop, b, kh);
      __builtin_amdgcn_s_setprio(1);
      qk(Sn, b ^ 1, kh);
      softmax_p(Sc, pb);
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) asm volatile("" ::"v"(pb[ct].x), "v"(pb[ct].y), "v"(pb[ct].z), "v"(pb[ct].w));
      __builtin_amdgcn_s_setprio(0);
      raise_max(Sc, pb);
      if (needs_mask(64 * (j + 1) + 32 * kh)) mask(Sn, 64 * (j + 1) + 32 * kh);
      __builtin_amdgcn_s_setprio(1);
      pv_mma(pb, vop);
      __builtin_amdgcn_s_setprio(0);
    }
    page_finish(raw, po_n);
    wait_loads();
    zero_v_tail(j + 1, b ^ 1);
    __syncthreads();
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) {
      po_v[pg] = po_k[pg];
      po_k[pg] = po_n[pg];
    }
  };
  if constexpr (KS == 2) {
    for (int j = 0; j < n_tiles; j += 2) {
      split_step(j, 0, S0, S1);
      if (j + 1 < n_tiles) split_step(j + 1, 1, S1, S0);
    }
    // Wave kh = 1 hands its state (reference max, row sums, accumulators) to
    // wave kh = 0 of its column group through LDS, free after the last
    // step's barrier; the receiver rescales both to the larger reference.
    static_assert((NW / KS) * (QT * 64 * 2 + QT * VD * 64 * 4) * 4 <= (int)sizeof(lds), "merge fits the tile buffers");
    float* xs = reinterpret_cast<float*>(lds) + cw * (QT * 64 * 2 + QT * VD * 64 * 4);
    if (kh == 1) {
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) {
        xs[ct * 64 + lane] = m[ct];
        xs[(QT + ct) * 64 + lane] = lsum[ct][0];
#pragma unroll
        for (int c = 0; c < VD; ++c)
          *reinterpret_cast<f32x4_t*>(xs + QT * 64 * 2 + ((ct * VD + c) * 64 + lane) * 4) = acc[ct][c];
      }
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) {
        const float m2 = xs[ct * 64 + lane];
        const float l2 = xs[(QT + ct) * 64 + lane];
        const float mm = fmax_prop(m[ct], m2);
        const float a1 = mm == kNegInf ? 0.f : fast_exp2(m[ct] - mm);
        const float a2 = mm == kNegInf ? 0.f : fast_exp2(m2 - mm);
        lsum[ct][0] = lsum[ct][0] * a1 + l2 * a2;
#pragma unroll
        for (int c = 0; c < VD; ++c) {
          const f32x4_t o2 = *reinterpret_cast<const f32x4_t*>(xs + QT * 64 * 2 + ((ct * VD + c) * 64 + lane) * 4);
          acc[ct][c] = acc[ct][c] * a1 + o2 * a2;
        }
      }
    }
  } else if (short_wg) {
    // Every tile is in LDS. The wave's last computed half forms no Sᵀ of the
    // half after it.
    half_step(0, S0, S1, 0, 1, 0, 0, 1 < wave_halves);
    half_step(1, S1, S0, 1, 0, 0, 1, 2 < wave_halves);
    half_step(2, S0, S1, 1, 1, 1, 0, 3 < wave_halves);
    half_step(3, S1, S0, 0, 0, 1, 1, false);
  } else {
    // Two tiles per iteration, so that buffer numbers are constants.
    for (int j = 0; j < n_tiles; j += 2) {
      tile_step(j, 0);
      if (j + 1 < n_tiles) tile_step(j + 1, 1);
    }
    // The last step's prefetch into LDS is still in flight: it must land
    // before the work-group ends and its LDS is handed to another.
    wait_loads();
  }

#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    const float lt = lsum[ct][0];
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    // acc[ct][c][i] is dim 16c + 4g + i. Lanes of 16-lane rows g and g^1 hold
    // the column's two 4-dim halves of each 8-dim group: one row swap per pair
    // of dim blocks (c, c+1) gives every lane 8 consecutive dims, stored as
    // 16 bytes: rows g even take block c at dims 16c + 4g, rows g odd block c+1
    // at dims 16(c+1) + 4(g-1).
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + (int64_t)(q_start + qi[ct]) * a.o_st +
                     (int64_t)(kvh * G + hl[ct]) * a.o_sh + 4 * g + 12 * (g & 1);
#pragma unroll
    for (int c = 0; c < VD; c += 2) {
      const uint32_t x0 = pack_bf16x2_hw(acc[ct][c][0] * inv, acc[ct][c][1] * inv);
      const uint32_t y0 = pack_bf16x2_hw(acc[ct][c][2] * inv, acc[ct][c][3] * inv);
      const uint32_t x1 = pack_bf16x2_hw(acc[ct][c + 1][0] * inv, acc[ct][c + 1][1] * inv);
      const uint32_t y1 = pack_bf16x2_hw(acc[ct][c + 1][2] * inv, acc[ct][c + 1][3] * inv);
      const auto sx = __builtin_amdgcn_permlane16_swap(x0, x1, false, false);
      const auto sy = __builtin_amdgcn_permlane16_swap(y0, y1, false, false);
      if (valid[ct] && kh == 0) st16(orow + 16 * c, make_uint4(sx[0], sy[0], sx[1], sy[1]));
    }
  }
  if (!MB) break;
  } while (--blk >= b_first);
}

// Decode view of a prefill batch: row b is sequence b; the decode work-group
// computes it only if it has exactly one query token.
static DecodeArgs single_query_view(const PrefillArgs& p) {
  DecodeArgs a{};
  a.q = p.q; a.q_sb = p.q_st; a.q_sh = p.q_sh;
  a.k_cache = p.k_cache; a.v_cache = p.v_cache;
  a.c_sb = p.c_sb; a.c_st = p.c_st; a.c_sh = p.c_sh;
  a.num_pages = p.num_pages;
  a.block_tables = p.block_tables; a.bt_stride = p.bt_stride; a.max_blocks = p.max_blocks;
  a.seq_lens = p.seq_lens;
  a.scale_log2 = p.scale_log2;
  a.out = p.out; a.o_sb = p.o_st; a.o_sh = p.o_sh;
  a.num_splits = 1; a.blocks_per_split = p.max_blocks;
  a.batch = p.num_seqs; a.num_heads = p.num_heads; a.num_kv_heads = p.num_kv_heads; a.head_dim = p.head_dim;
  a.waves = kDecodeWaves;
  a.query_start_loc = p.query_start_loc;
  a.context_lens = p.context_lens;
  return a;
}

// Launch geometry of a prefill batch for CB columns ((query, head) pairs of
// one KV head) per work-group.
struct PrefillGrid {
  int64_t bound = 0;  // query-block numbers
  int dense_qb = 0;   // > 0: dense numbering with this many blocks per sequence
  int xcd_group = 0;
  int64_t per_xcd = 0;
  int64_t prefill_wgs = 0, dec_wgs = 0;
};

static PrefillGrid plan_prefill(const PrefillArgs& a, int64_t CB) {
  PrefillGrid p;
  const int64_t G = a.num_heads / a.num_kv_heads;
  // Upper bound of the block count: Σ ceil(G·q_s / CB) ≤ (G·T + S·(CB-1)) / CB
  // over the sequences the prefill work-groups compute.
  int64_t T = a.num_tokens, S = a.num_seqs;
  if (a.single_query_seqs > 0) {
    T -= a.single_query_seqs;
    S -= a.single_query_seqs;
  }
  p.bound = S > 0 ? (G * T + S * (CB - 1)) / CB : 0;
  // Blocks are numbered densely (ceil(G·max_query_len / CB) per sequence,
  // found by division) unless that wastes more than a quarter of the grid on
  // empty blocks, as in a mixed step; then compactly (found by a scan).
  const int64_t dense = (G * a.max_query_len + CB - 1) / CB;
  if (dense * a.num_seqs * 4 <= p.bound * 5) {
    p.dense_qb = (int)dense;
    p.bound = dense * a.num_seqs;
  }
  p.xcd_group = (a.num_kv_heads <= 8 && 8 % a.num_kv_heads == 0) ? 8 / a.num_kv_heads : 0;
  if (p.dense_qb > 0 && (int64_t)a.num_seqs * a.num_kv_heads >= 64) p.xcd_group = -1;
  p.per_xcd = (p.bound * a.num_kv_heads + 7) / 8;
  p.prefill_wgs = p.xcd_group > 0 ? 8 * ((p.bound + p.xcd_group - 1) / p.xcd_group)
                  : p.xcd_group < 0 ? 8 * p.per_xcd
                                    : p.bound * a.num_kv_heads;
  // Decode work-groups: one per (sequence, column group), rounded up to whole XCD rounds.
  p.dec_wgs = a.single_query_seqs != 0 ? ((int64_t)a.num_seqs * a.num_kv_heads * ((G + 15) / 16) + 7) / 8 * 8 : 0;
  return p;
}

template <int D, int NW, int QT, int KS = 1>
static hipError_t launch_prefill(const PrefillArgs& a, const PrefillGrid& p, int bpw, hipStream_t stream) {
  if (p.prefill_wgs + p.dec_wgs == 0) return hipSuccess;
  if (p.prefill_wgs + p.dec_wgs > 0x7ffffff0) return hipErrorInvalidValue;
  if constexpr (KS == 1) {
    if (bpw > 1) {
      hipLaunchKernelGGL((paged_prefill_kernel<D, NW, QT, true, 1>), dim3((unsigned)(p.dec_wgs + p.prefill_wgs)),
                         dim3(NW * 64), 0, stream, a, (int)p.bound, p.dense_qb, p.xcd_group, (int)p.per_xcd,
                         single_query_view(a), (int)p.dec_wgs, bpw);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((paged_prefill_kernel<D, NW, QT, false, KS>), dim3((unsigned)(p.dec_wgs + p.prefill_wgs)),
                     dim3(NW * 64), 0, stream, a, (int)p.bound, p.dense_qb, p.xcd_group, (int)p.per_xcd,
                     single_query_view(a), (int)p.dec_wgs, 1);
  return hipGetLastError();
}

// Blocks per work-group: when every sequence's keys fit two 64-key tiles
// (table width ≤ 8 pages) and the one-block grid is more than one round of
// two work-groups per CU, a work-group takes several blocks of one (sequence,
// KV head), which read the same tiles: the fewest per work-group that make
// the grid one round (64 x 128: 4 blocks per work-group, 512 work-groups).
// The tuning switch kTunePrefillBlocksPerWg overrides the choice when the
// table width allows it.
static int prefill_blocks_per_wg(const PrefillArgs& a, const PrefillGrid& p1) {
  if (a.max_blocks > 8) return 1;
  const int forced = tuning(kTunePrefillBlocksPerWg);
  if (forced > 0) return forced;
  if (p1.dense_qb <= 1) return 1;
  const int64_t slots = 2 * (int64_t)device_cus();
  const int64_t pairs = (int64_t)a.num_seqs * a.num_kv_heads;
  const int64_t per_pair = slots / pairs;  // work-groups per (sequence, KV head) in one round
  if (per_pair >= p1.dense_qb) return 1;
  if (per_pair == 0) return p1.dense_qb;
  return (int)((p1.dense_qb + per_pair - 1) / per_pair);
}

// Two column tiles per wave (128 columns per work-group) unless that grid
// gives fewer than two prefill work-groups per CU (short batches, mixed
// steps): then 64 columns per work-group, twice the work-groups, computed by
// the key split (two column groups of two waves, each wave on one half of
// every key tile; 8 x (1024 + 128): 29.4-29.9 us against 31.3-31.7 us for one
// column tile per wave over every key, the choice behind the tuning switch
// kTunePrefillShortGrid; mixed 1 x 512 + 63 decodes: 29.3-30.0 us either way).
template <int D>
static hipError_t prefill_for_dim(const PrefillArgs& a, hipStream_t stream) {
  const PrefillGrid p2 = plan_prefill(a, 4 * 2 * 16);
  if (p2.prefill_wgs >= 2 * (int64_t)device_cus()) {
    const int bpw = prefill_blocks_per_wg(a, p2);
    if (bpw == 1) return launch_prefill<D, 4, 2>(a, p2, 1, stream);
    return launch_prefill<D, 4, 2>(a, plan_prefill(a, 4 * 2 * 16 * (int64_t)bpw), bpw, stream);
  }
  if (tuning(kTunePrefillShortGrid) == 1) return launch_prefill<D, 4, 1>(a, plan_prefill(a, 4 * 1 * 16), 1, stream);
  return launch_prefill<D, 4, 2, 2>(a, plan_prefill(a, 4 / 2 * 2 * 16), 1, stream);
}

hipError_t paged_prefill(const PrefillArgs& a, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return prefill_for_dim<64>(a, stream);
    case 128: return prefill_for_dim<128>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
