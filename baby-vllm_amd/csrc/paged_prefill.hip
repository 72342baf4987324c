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
//                                         Sᵀ registers, Vᵀ element-picked from LDS rows)
// Keys at or past hi = min(seq_len, ctx + last query + 1) are staged as zeros,
// so cache slots that were never written (possibly NaN) never reach a product.
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

template <int D, int NW, int QT>
__global__ __launch_bounds__(NW * 64, 2) void paged_prefill_kernel(PrefillArgs a, int n_qb, int total_wg,
                                                                  int per_xcd) {
  constexpr int KT = 64;
  constexpr int PITCH = D + 8;  // bf16 elements; 16-byte pad keeps 16-row column reads conflict-free
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int OD = D / 4;
  constexpr int CPR = D / 8;
  constexpr int CHUNKS = KT * CPR;
  constexpr int PER_T = CHUNKS / (NW * 64);
  static_assert(PER_T * NW * 64 == CHUNKS, "tile chunks must divide evenly over the work-group");
  static_assert(KT == 64, "a key tile spans four 16-token pages");
  typedef typename std::conditional<VD == 8, uint4, uint2>::type VRow;

  __shared__ __attribute__((aligned(16))) uint16_t lds_k[2][KT * PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t lds_v[2][KT * PITCH];

  // Work-groups are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous range of (sequence, KV head, query block) so the query blocks
  // that share a prefix also share an L2.
  const int id = blockIdx.x;
  const int L = (id & 7) * per_xcd + (id >> 3);
  if (L >= total_wg) return;
  const int qb = n_qb - 1 - (L % n_qb);  // later (longer) query blocks first
  const int sk = L / n_qb;
  const int kvh = sk % a.num_kv_heads;
  const int s = sk / a.num_kv_heads;

  const int G = a.num_heads / a.num_kv_heads;
  const int QP = 16 / G;
  const int QB = NW * QT * QP;
  const int q_start = uniform(a.query_start_loc[s]);
  const int q_len = uniform(a.query_start_loc[s + 1]) - q_start;
  if (qb * QB >= q_len) return;
  if (q_len == 1 && a.single_query_seqs != 0) return;  // on the decode kernel
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

  // The four page numbers of a key tile are fetched first, as scalar loads
  // (constant address space, counted apart from the vector loads), and then all
  // data loads of the tile are issued back to back.
  typedef const int32_t __attribute__((address_space(4)))* ConstI32;
  const ConstI32 bts = (ConstI32)bt;
  constexpr int PAGES_PER_TILE = KT / 16;
  uint4 stk[PER_T], stv[PER_T];
  auto stage_load = [&](int kt) {
    int64_t page_off[PAGES_PER_TILE];
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) {
      int phys = bts[min(kt * PAGES_PER_TILE + pg, a.max_blocks - 1)];
      phys = min(max(phys, 0), a.num_pages - 1);
      page_off[pg] = (int64_t)phys * a.c_sb;
    }
    // Keep the four table loads together ahead of the data loads (the compiler
    // would otherwise sink each into the branch that uses it, one wait apiece).
#pragma unroll
    for (int pg = 0; pg < PAGES_PER_TILE; ++pg) asm volatile("" ::"s"(page_off[pg]));
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int e = threadIdx.x + r * NW * 64;
      const int key = e / CPR;
      const int part = e - key * CPR;
      const int pos = kt * KT + key;
      if (pos < hi) {
        const int pg = key >> 4;  // selects instead of a dynamically indexed private array
        const int64_t po = pg == 0 ? page_off[0] : pg == 1 ? page_off[1] : pg == 2 ? page_off[2] : page_off[3];
        const int64_t off = po + (int64_t)(pos & 15) * a.c_st + part * 8;
        stk[r] = ld16(kc + off);
        stv[r] = ld16(vc + off);
      } else {
        stk[r] = make_uint4(0, 0, 0, 0);
        stv[r] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto stage_store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int e = threadIdx.x + r * NW * 64;
      const int key = e / CPR;
      const int part = e - key * CPR;
      st16(&lds_k[buf][key * PITCH + part * 8], stk[r]);
      st16(&lds_v[buf][key * PITCH + part * 8], stv[r]);
    }
  };

  if (n_tiles > 0) {
    stage_load(0);
    stage_store(0);
  }
  __syncthreads();

  // Staging runs on every iteration, also the last: tile n_tiles lies wholly at
  // or past hi, so it issues no data load and stores zeros into the idle
  // buffer. Branching on kt + 1 < n_tiles instead would leave the loads looking
  // pending at the loop header, and the compiler would drain them there.
  for (int kt = 0; kt < n_tiles; ++kt) {
    const int buf = kt & 1;
    stage_load(kt + 1);

    if (wave_live && kt * KT <= wave_hi) {
      const uint16_t* K = lds_k[buf];
      const uint16_t* V = lds_v[buf];
      f32x4_t sacc[QT][4];
#pragma unroll
      for (int ct = 0; ct < QT; ++ct)
#pragma unroll
        for (int t = 0; t < 4; ++t) sacc[ct][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          const uint4 ka = ld16(K + (16 * t + n) * PITCH + 8 * (4 * c + g));
#pragma unroll
          for (int ct = 0; ct < QT; ++ct) sacc[ct][t] = mfma_16x16x32(ka, qreg[ct][c], sacc[ct][t]);
        }
      }

      uint4 pb[QT][2];
      // Some key of the tile may be invisible to some column: past the causal
      // diagonal of the wave's first query, or at/after hi.
      const bool diag = (kt * KT + KT - 1 > ctx + wave_q0) || (kt * KT + KT > hi);
#pragma unroll
      for (int ct = 0; ct < QT; ++ct) {
        float sv[4][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[t][i] = sacc[ct][t][i] * a.scale_log2;
        if (diag) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int pos = kt * KT + 16 * t + 4 * g + i;
              if (pos > qpos[ct] || pos >= hi) sv[t][i] = kNegInf;
            }
        }
        float mx = kNegInf;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          mx = fmaxf(mx, fmaxf(fmaxf(sv[t][0], sv[t][1]), fmaxf(sv[t][2], sv[t][3])));
        mx = max_across_groups(mx);
        const float m_new = fmaxf(m[ct], mx);
        const float alpha = fast_exp2(m[ct] - m_new);
        float p[4][4];
        float psum = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[t][i] = fast_exp2(sv[t][i] - m_new);
            psum += p[t][i];
          }
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

#pragma unroll
      for (int u = 0; u < 2; ++u) {
        VRow vr[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = 16 * (2 * u + j / 4) + 4 * g + (j & 3);
          if constexpr (VD == 8) vr[j] = ld16(V + key * PITCH + VD * n);
          else vr[j] = ld8(V + key * PITCH + VD * n);
        }
#pragma unroll
        for (int c = 0; c < VD; ++c) {
          uint32_t d[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const uint32_t* r0 = reinterpret_cast<const uint32_t*>(&vr[2 * jj]);
            const uint32_t* r1 = reinterpret_cast<const uint32_t*>(&vr[2 * jj + 1]);
            d[jj] = pick_halves(r0[c / 2], r1[c / 2], c & 1);
          }
          const uint4 va = make_uint4(d[0], d[1], d[2], d[3]);
#pragma unroll
          for (int ct = 0; ct < QT; ++ct) acc[ct][c] = mfma_16x16x32(va, pb[ct][u], acc[ct][c]);
        }
      }
    }

    stage_store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int ct = 0; ct < QT; ++ct) {
    const float lt = sum_across_groups(l[ct]);
    if (!valid[ct]) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + (int64_t)(q_start + qi[ct]) * a.o_st +
                     (int64_t)(kvh * G + hl) * a.o_sh + OD * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (VD == 8) {
        uint4 pk;
        pk.x = pack_bf16x2_hw(acc[ct][0][i] * inv, acc[ct][1][i] * inv);
        pk.y = pack_bf16x2_hw(acc[ct][2][i] * inv, acc[ct][3][i] * inv);
        pk.z = pack_bf16x2_hw(acc[ct][4][i] * inv, acc[ct][5][i] * inv);
        pk.w = pack_bf16x2_hw(acc[ct][6][i] * inv, acc[ct][7][i] * inv);
        st16(orow + VD * i, pk);
      } else {
        uint2 pk;
        pk.x = pack_bf16x2_hw(acc[ct][0][i] * inv, acc[ct][1][i] * inv);
        pk.y = pack_bf16x2_hw(acc[ct][2][i] * inv, acc[ct][3][i] * inv);
        st8(orow + VD * i, pk);
      }
    }
  }
}

template <int D, int NW, int QT>
static hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  const int G = a.num_heads / a.num_kv_heads;
  const int QB = NW * QT * (16 / G);
  const int n_qb = (a.max_query_len + QB - 1) / QB;
  const int64_t total = (int64_t)n_qb * a.num_kv_heads * a.num_seqs;
  if (total == 0) return hipSuccess;
  if (total > 0x7ffffff0) return hipErrorInvalidValue;
  const int per_xcd = (int)((total + 7) / 8);
  hipLaunchKernelGGL((paged_prefill_kernel<D, NW, QT>), dim3((unsigned)(8 * per_xcd)), dim3(NW * 64), 0,
                     stream, a, n_qb, (int)total, per_xcd);
  return hipGetLastError();
}

// Sequences with a single query token (decode rows of a mixed step) go to the
// decode kernel, whose waves split the row's pages; the prefill kernel would
// walk them with one live wave per work-group.
hipError_t paged_prefill(const PrefillArgs& a, hipStream_t stream) {
  if (a.single_query_seqs != 0) {
    const hipError_t e = decode_single_query_seqs(a, stream);
    if (e != hipSuccess || a.single_query_seqs == a.num_seqs) return e;
  }
  switch (a.head_dim) {
    case 64: return launch_prefill<64, 4, 2>(a, stream);
    case 128: return launch_prefill<128, 4, 2>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
