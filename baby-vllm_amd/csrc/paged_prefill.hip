// Varlen paged prefill attention: causal GQA attention for a flattened batch of
// sequences whose keys/values (cached prefix + the step's new tokens) are read
// straight from the paged cache through the block table.
//
// Replaces paged_prefill_attn_kernel (babyvllm/kernels/paged_prefill.py:6-101).
//
// Work-group = (sequence, KV head, block of QB query rows). All G query heads
// of the KV head are packed into the MFMA column dimension, so every K/V tile
// is staged once per work-group and shared by the whole GQA group:
//   column n of a 16-column tile = (query n / G, head n % G), n < (16 / G)·G.
// Each of the NW waves owns QT such column tiles; QB = NW·QT·(16/G).
// Keys are processed in tiles of 64 (four 16-token pages) staged in LDS, double
// buffered: the global loads of tile t+1 are in flight while tile t computes.
//   Sᵀ[16 keys × 16 cols] = K · Qᵀ       (mfma 16x16x32, K operand from LDS)
//   Oᵀ[D × 16 cols]      += Vᵀ · Pᵀ      (mfma 16x16x32 over 32 keys, Pᵀ from the
//                                         Sᵀ registers, Vᵀ by LDS transpose reads)
// Keys at or past hi = min(seq_len, ctx + last query + 1) are staged as zeros,
// so cache slots that were never written (possibly NaN) never reach a product.
//
// Sequences with a single query token (the decode rows of a mixed step) are
// instead computed by decode work-groups (paged_decode_wg.h) placed in front of
// the prefill work-groups of the same launch: their waves split a row's pages,
// where a prefill work-group would walk them with one live wave.
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"
#include "paged_decode_wg.h"

namespace bvllm {

// Query blocks of QB rows are numbered sequence by sequence, the blocks of a
// sequence last (most keys) first; a sequence with one query token has none
// when the decode work-groups compute it. Finds the sequence s and block qb of
// number r, or returns false if r is past the last block. Every wave computes
// the same wave-uniform answer (a scan of the per-sequence block counts).
__device__ __forceinline__ bool find_query_block(const PrefillArgs& a, int QB, int r, int& s_out, int& qb_out) {
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
        nb[c] = (ql == 1 && a.single_query_seqs != 0) ? 0 : (ql + QB - 1) / QB;
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

// Waves and pages in flight of the decode work-groups of a mixed step.
constexpr int kDecodeWaves = 4;
constexpr int kDecodeDepth = 2;

template <int D, int NW, int QT>
__global__ __launch_bounds__(NW * 64, 2) void paged_prefill_kernel(PrefillArgs a, int n_blocks_bound, int dense_qb,
                                                                  int xcd_group, int per_xcd, DecodeArgs dec,
                                                                  int n_dec_wgs) {
  constexpr int KT = 64;
  // LDS row pitches (bf16 elements): K rows are read 16 B per lane from 16
  // rows (a 16-byte pad spreads them over all banks); V rows are read by
  // transpose reads, 32 B from each of 4 rows per 16 lanes (a 32-byte pad).
  constexpr int PITCH = D + 8;
  constexpr int PITCH_V = D + 16;
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int CPR = D / 8;
  constexpr int CHUNKS = KT * CPR;
  constexpr int PER_T = CHUNKS / (NW * 64);
  static_assert(PER_T * NW * 64 == CHUNKS, "tile chunks must divide evenly over the work-group");
  static_assert(KT == 64, "a key tile spans four 16-token pages");

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * KT * PITCH + 2 * KT * PITCH_V];
  uint16_t (*lds_k)[KT * PITCH] = reinterpret_cast<uint16_t (*)[KT * PITCH]>(lds);
  uint16_t (*lds_v)[KT * PITCH_V] = reinterpret_cast<uint16_t (*)[KT * PITCH_V]>(lds + 2 * KT * PITCH);
  static_assert(NW == kDecodeWaves, "decode work-groups run with the prefill work-group size");
  static_assert(decode_lds_bytes<D, kDecodeWaves>(16) <= sizeof(lds), "decode work-group LDS");

  // The first n_dec_wgs work-groups (a multiple of 8) are decode work-groups,
  // one per (sequence, KV head); those past the batch have nothing to do.
  if ((int)blockIdx.x < n_dec_wgs) {
    if ((int)blockIdx.x < dec.batch * dec.num_kv_heads)
      decode_work_group<D, kDecodeWaves, kDecodeDepth>(dec, blockIdx.x, reinterpret_cast<float*>(lds));
    return;
  }

  const int G = a.num_heads / a.num_kv_heads;
  const int QP = 16 / G;
  const int QB = NW * QT * QP;

  // Work-groups are dispatched round-robin over the 8 XCDs (XCD = id mod 8).
  // xcd_group == -1 (many (sequence, KV head) pairs, dense numbering): each XCD
  // takes a contiguous range of (sequence, KV head, block), so the blocks that
  // share a prefix share an L2 and every XCD gets many whole pairs.
  // xcd_group = 8 / Hkv > 0 (few pairs, or a mixed step): KV head h is served
  // by XCDs h·xcd_group .. +xcd_group-1, which deal its query blocks out in
  // boustrophedon order (0 1 | 1 0 | 0 1 ...): each L2 holds one KV head's
  // keys, and the heavy-to-light run of a sequence's blocks spreads evenly.
  const int id = blockIdx.x - n_dec_wgs;
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
  } else if (!find_query_block(a, QB, r, s, qb)) {
    return;
  }
  const int q_start = uniform(a.query_start_loc[s]);
  const int q_len = uniform(a.query_start_loc[s + 1]) - q_start;
  if (qb * QB >= q_len) return;
  if (q_len == 1 && a.single_query_seqs != 0) return;  // on the decode work-groups
  const int seq_len = uniform(a.seq_lens[s]);
  const int ctx = uniform(a.context_lens[s]);
  const int q_last = min(q_len, (qb + 1) * QB) - 1;
  const int hi = min(seq_len, ctx + q_last + 1);
  const int n_tiles = hi > 0 ? (hi + KT - 1) / KT : 0;

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;
  const int w = wave_id();
  const int qi_in = n / G;
  const int hl = n - qi_in * G;
  const bool col_ok = n < QP * G;

  const int wave_q0 = qb * QB + w * QT * QP;  // first query index of this wave
  const bool wave_live = wave_q0 < q_len;
  const int wave_hi = ctx + min(q_len - 1, wave_q0 + QT * QP - 1);  // last visible key position

  int qi[QT];
  int qpos[QT];
  bool valid[QT];
  uint4 qreg[QT][KC];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    qi[ct] = wave_q0 + ct * QP + qi_in;
    valid[ct] = col_ok && qi[ct] < q_len;
    qpos[ct] = valid[ct] ? ctx + qi[ct] : 0x7fffffff;
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)(q_start + qi[ct]) * a.q_st +
                           (int64_t)(kvh * G + hl) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      qreg[ct][c] = valid[ct] ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }

  // Make the Q loads complete here, once: otherwise they look pending at the
  // key loop's header and the compiler drains every load there, including the
  // next tile's staging loads, on each iteration.
#pragma unroll
  for (int ct = 0; ct < QT; ++ct)
#pragma unroll
    for (int c = 0; c < KC; ++c) asm volatile("" ::"v"(qreg[ct][c].x), "v"(qreg[ct][c].y), "v"(qreg[ct][c].z), "v"(qreg[ct][c].w));

  float m[QT], l[QT];
  f32x4_t acc[QT][VD];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    m[ct] = kNegInf;
    l[ct] = 0.f;
#pragma unroll
    for (int c = 0; c < VD; ++c) acc[ct][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;
  const int32_t* bt = a.block_tables + (int64_t)s * a.bt_stride;

  // Staging. Chunk e = threadIdx.x + r·NW·64 (r < PER_T) of a 64-key tile is
  // key e / CPR, 16-byte part e % CPR. Tiles start on page boundaries, so the
  // chunk's byte offset inside its page is the same on every tile, and the 64
  // chunks of one wave lie in one page: each load takes the page base as a
  // scalar operand plus a loop-invariant offset. Page numbers are clamped into
  // the pool, so every staging load is in bounds, keys at or past hi included;
  // V rows of those keys are replaced by zeros before they reach LDS (unwritten
  // slots may hold NaN, and 0·NaN would poison the PV product), K rows of those
  // keys only reach scores that the mask replaces by -inf.
  static_assert(16 % (64 / CPR) == 0, "a wave's staging chunks must lie in one page");
  constexpr int PAGES_PER_TILE = KT / 16;
  // Chunk e lies in page e / (16·CPR) = e / (2D) of the tile: page
  // r·PG_STEP + (wave's offset), known at compile time up to the wave.
  constexpr int PG_STEP = NW * 64 / (2 * D);
  static_assert(PG_STEP * 2 * D == NW * 64 && PG_STEP * PER_T == PAGES_PER_TILE, "staging page layout");
  static_assert(PG_STEP == 1 || PG_STEP == 2, "a wave's chunks of one r lie in page r·PG_STEP + (0 or 1)");
  const int pg_wave = uniform((int)(threadIdx.x / (2 * D)));  // always 0 when PG_STEP == 1
  uint32_t st_off[PER_T];  // byte offset of the chunk inside its page
  int st_key[PER_T];       // key of the chunk within the tile
#pragma unroll
  for (int r = 0; r < PER_T; ++r) {
    const int e = threadIdx.x + r * NW * 64;
    const int key = e / CPR;
    const int part = e - key * CPR;
    st_key[r] = key;
    st_off[r] = (uint32_t)(((int64_t)(key & 15) * a.c_st + part * 8) * 2);
  }

  // The four page numbers of a tile, as scalar loads (constant address space)
  // issued together and consumed together: one wait for all four. Entries
  // past the row's last table entry are clamped to it (only the last tiles
  // reach there).
  typedef const int32_t __attribute__((address_space(4)))* ConstI32;
  const ConstI32 bts = (ConstI32)bt;
  const uint32_t page_elems = (uint32_t)a.c_sb;  // < 2^31, checked on the host
  auto page_bases = [&](int kt, int64_t (&po)[PAGES_PER_TILE]) {
    int raw[PAGES_PER_TILE];
    const int i0 = kt * PAGES_PER_TILE;
    if (i0 + PAGES_PER_TILE <= a.max_blocks) {
#pragma unroll
      for (int pg = 0; pg < PAGES_PER_TILE; ++pg) raw[pg] = bts[i0 + pg];
    } else {
#pragma unroll
      for (int pg = 0; pg < PAGES_PER_TILE; ++pg) raw[pg] = bts[min(i0 + pg, a.max_blocks - 1)];
    }
    asm volatile("" ::"s"(raw[0]), "s"(raw[1]), "s"(raw[2]), "s"(raw[3]));
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg)
      po[pg] = (int64_t)((uint64_t)(uint32_t)min(max(raw[pg], 0), a.num_pages - 1) * page_elems);
  };
  static_assert(PAGES_PER_TILE == 4, "page_bases consumes four entries");

  // Staging loads are inline-asm global loads, waited for explicitly before
  // their registers are stored to LDS: the compiler's own waitcnt insertion
  // would drain them at the loop header, serialising the next tile's memory
  // latency with the current tile's compute.
  u32x4_t stk[PER_T], stv[PER_T];
  auto stage_issue = [&](const int64_t (&po)[PAGES_PER_TILE]) {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      int64_t p;
      if constexpr (PG_STEP == 1) p = po[r];
      else p = pg_wave ? po[PG_STEP * r + 1] : po[PG_STEP * r];
      const uint16_t* kb = kc + p;
      const uint16_t* vb = vc + p;
      asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(stk[r]) : "v"(st_off[r]), "s"(kb));
      asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(stv[r]) : "v"(st_off[r]), "s"(vb));
    }
  };
  // Waits for the staging loads of tile kt, zeroes its V rows at or past hi and
  // stores the tile into LDS buffer buf.
  auto stage_finish = [&](int kt, int buf) {
    if constexpr (PER_T == 4)
      asm volatile("s_waitcnt vmcnt(0)"
                   : "+v"(stk[0]), "+v"(stk[1]), "+v"(stk[2]), "+v"(stk[3]),
                     "+v"(stv[0]), "+v"(stv[1]), "+v"(stv[2]), "+v"(stv[3]));
    else
      asm volatile("s_waitcnt vmcnt(0)" : "+v"(stk[0]), "+v"(stk[1]), "+v"(stv[0]), "+v"(stv[1]));
    static_assert(PER_T == 4 || PER_T == 2, "staging wait covers 2 or 4 chunks");
    if (kt * KT + KT > hi) {  // the tile reaches hi (uniform)
#pragma unroll
      for (int r = 0; r < PER_T; ++r)
        if (kt * KT + st_key[r] >= hi) stv[r] = u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int e = threadIdx.x + r * NW * 64;
      const int part = e - st_key[r] * CPR;
      *reinterpret_cast<u32x4_t*>(&lds_k[buf][st_key[r] * PITCH + part * 8]) = stk[r];
      *reinterpret_cast<u32x4_t*>(&lds_v[buf][st_key[r] * PITCH_V + part * 8]) = stv[r];
    }
  };

  // Last visible key of each column (its query position, at most hi - 1):
  // on tiles that reach past a column's diagonal or past hi, key pos is masked
  // for the column iff pos > lim.
  int lim[QT];
#pragma unroll
  for (int ct = 0; ct < QT; ++ct) lim[ct] = min(qpos[ct], hi - 1);

  int64_t po[PAGES_PER_TILE];
  if (n_tiles > 0) {
    page_bases(0, po);
    stage_issue(po);
    stage_finish(0, 0);
  }
  __syncthreads();

  // One key tile: stage tile kt + 1 into the idle buffer while tile kt computes.
  // Staging runs on every tile, also the last: tile n_tiles is clamped into the
  // pool like any other and its buffer is never read.
  auto tile = [&](const int kt, const int buf) {
    page_bases(kt + 1, po);
    stage_issue(po);

    if (wave_live && kt * KT <= wave_hi) {
      const uint16_t* K = lds_k[buf];
      const uint16_t* V = lds_v[buf];
      f32x4_t sacc[QT][4];
#pragma unroll
      for (int ct = 0; ct < QT; ++ct)
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[ct][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      // The MFMA runs are issued at raised wave priority: the SIMD's other wave
      // (another work-group's, usually in its softmax) fills the VALU slots
      // between them instead of delaying them.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const uint4 ka = ld16(K + (16 * t + n) * PITCH + 8 * (4 * c + g));
#pragma unroll
          for (int ct = 0; ct < QT; ++ct) sacc[ct][t] = mfma_16x16x32(ka, qreg[ct][c], sacc[ct][t]);
        }
      }

      __builtin_amdgcn_s_setprio(0);
      uint4 pb[QT][2];
      // Some key of the tile may be invisible to some column: past the causal
      // diagonal of the wave's first query, or at/after hi.
      const bool diag = (kt * KT + KT - 1 > ctx + wave_q0) || (kt * KT + KT > hi);
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) {
        // Raw scores; the scale (> 0, so the max commutes with it) is applied
        // inside the exponent's fma: p = 2^(s·scale_log2 − m).
        float sv[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[t][i] = sacc[ct][t][i];
        if (diag) {
          // key 16t + 4g + i of the tile is masked iff 16t + i > lim - kt·KT - 4g.
          const int rel = lim[ct] - kt * KT - 4 * g;
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (16 * t + i > rel) sv[t][i] = kNegInf;
        }
        float mx = kNegInf;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          mx = fmax_prop(mx, fmax_prop(fmax_prop(sv[t][0], sv[t][1]), fmax_prop(sv[t][2], sv[t][3])));
        mx = max_across_groups(mx);
        const float m_new = fmax_prop(m[ct], mx * a.scale_log2);
        const float alpha = fast_exp2(m[ct] - m_new);
        float p[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) p[t][i] = fast_exp2(__builtin_fmaf(sv[t][i], a.scale_log2, -m_new));
        float ps[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) ps[t] = (p[t][0] + p[t][1]) + (p[t][2] + p[t][3]);
        const float psum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
        l[ct] = l[ct] * alpha + psum;
        m[ct] = m_new;
        if (!wave_all_one(alpha)) {  // x·1 == x: skipping is exact
#pragma unroll
          for (int c = 0; c < VD; ++c) acc[ct][c] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          pb[ct][u].x = pack_bf16x2_hw(p[2 * u][0], p[2 * u][1]);
          pb[ct][u].y = pack_bf16x2_hw(p[2 * u][2], p[2 * u][3]);
          pb[ct][u].z = pack_bf16x2_hw(p[2 * u + 1][0], p[2 * u + 1][1]);
          pb[ct][u].w = pack_bf16x2_hw(p[2 * u + 1][2], p[2 * u + 1][3]);
        }
      }

      // Vᵀ operand of dims 16c .. 16c+15 over keys 32u + {4g .. 4g+3, 16+4g .. 16+4g+3}
      // (the keys whose P this lane holds): two transpose reads.
      const int trow = 4 * g + (n >> 2);
      const int tcol = 4 * (n & 3);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int c = 0; c < VD; ++c) {
          const uint2 lo = ld_tr16(V + (32 * u + trow) * PITCH_V + 16 * c + tcol);
          const uint2 hi2 = ld_tr16(V + (32 * u + 16 + trow) * PITCH_V + 16 * c + tcol);
          const uint4 va = make_uint4(lo.x, lo.y, hi2.x, hi2.y);
#pragma unroll
          for (int ct = 0; ct < QT; ++ct) acc[ct][c] = mfma_16x16x32(va, pb[ct][u], acc[ct][c]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }

    stage_finish(kt + 1, buf ^ 1);
    __syncthreads();
  };

  // Two tiles per iteration, so that each tile's LDS buffer is a constant.
  for (int kt = 0; kt < n_tiles; kt += 2) {
    tile(kt, 0);
    if (kt + 1 < n_tiles) tile(kt + 1, 1);
  }

#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    const float lt = sum_across_groups(l[ct]);
    if (!valid[ct]) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    // acc[ct][c][i] is dim 16c + 4g + i.
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + (int64_t)(q_start + qi[ct]) * a.o_st +
                     (int64_t)(kvh * G + hl) * a.o_sh + 4 * g;
#pragma unroll
    for (int c = 0; c < VD; ++c) {
      uint2 pk;
      pk.x = pack_bf16x2_hw(acc[ct][c][0] * inv, acc[ct][c][1] * inv);
      pk.y = pack_bf16x2_hw(acc[ct][c][2] * inv, acc[ct][c][3] * inv);
      st8(orow + 16 * c, pk);
    }
  }
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
  a.splits_per_wg = 1;
  a.query_start_loc = p.query_start_loc;
  a.context_lens = p.context_lens;
  return a;
}

template <int D, int NW, int QT>
static hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  const int G = a.num_heads / a.num_kv_heads;
  const int64_t QB = NW * QT * (16 / G);
  // Upper bound of the query-block count: Σ ceil(q_s / QB) ≤ (T + S·(QB-1)) / QB
  // over the sequences the prefill work-groups compute.
  int64_t T = a.num_tokens, S = a.num_seqs;
  if (a.single_query_seqs > 0) {
    T -= a.single_query_seqs;
    S -= a.single_query_seqs;
  }
  int64_t bound = S > 0 ? (T + S * (QB - 1)) / QB : 0;
  // Query blocks are numbered densely (ceil(max_query_len / QB) per sequence,
  // found by division) unless that wastes more than a quarter of the grid on
  // empty blocks, as in a mixed step; then compactly (found by a scan).
  const int64_t dense = (a.max_query_len + QB - 1) / QB;
  int dense_qb = 0;
  if (dense * a.num_seqs * 4 <= bound * 5) {
    dense_qb = (int)dense;
    bound = dense * a.num_seqs;
  }
  int xcd_group = (a.num_kv_heads <= 8 && 8 % a.num_kv_heads == 0) ? 8 / a.num_kv_heads : 0;
  if (dense_qb > 0 && (int64_t)a.num_seqs * a.num_kv_heads >= 64) xcd_group = -1;
  const int64_t per_xcd = (bound * a.num_kv_heads + 7) / 8;
  const int64_t prefill_wgs = xcd_group > 0 ? 8 * ((bound + xcd_group - 1) / xcd_group)
                              : xcd_group < 0 ? 8 * per_xcd
                                              : bound * a.num_kv_heads;
  const int64_t dec_wgs = a.single_query_seqs != 0 ? ((int64_t)a.num_seqs * a.num_kv_heads + 7) / 8 * 8 : 0;
  if (prefill_wgs + dec_wgs == 0) return hipSuccess;
  if (prefill_wgs + dec_wgs > 0x7ffffff0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_prefill_kernel<D, NW, QT>), dim3((unsigned)(dec_wgs + prefill_wgs)), dim3(NW * 64), 0,
                     stream, a, (int)bound, dense_qb, xcd_group, (int)per_xcd, single_query_view(a),
                     (int)dec_wgs);
  return hipGetLastError();
}

hipError_t paged_prefill(const PrefillArgs& a, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return launch_prefill<64, 4, 2>(a, stream);
    case 128: return launch_prefill<128, 4, 2>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
