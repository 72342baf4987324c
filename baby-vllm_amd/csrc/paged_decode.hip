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
// Per page (16 tokens) and wave, both products run on bf16 MFMA:
//   Sᵀ[16 tok × 16 col] = K[16 tok × D] · Qᵀ[D × 16 col]   (D/32 × mfma 16x16x32)
//     col n < G is query head kvh·G + n (the GQA group), the rest is zero padding.
//     Lane (n + 16g) loads K row n, dims 8(4c+g)..+8 for c < D/32 (16-byte loads);
//     the result lane (n + 16g) holds S[head n][token 4g+i], i < 4.
//   Oᵀ[D × 16 col] += Vᵀ[D × 16 tok] · Pᵀ[16 tok × 16 col]  (D/16 × mfma 16x16x16)
//     P comes straight from the Sᵀ registers (same lane layout as the B operand);
//     lane (m + 16g) loads V rows 4g..4g+3, dims (D/16)·m..+D/16 (one 16-byte load
//     per row at D = 128), and MFMA c takes element c of those rows, so MFMA c's
//     output row r is dim (D/16)·r + c. Lane (n + 16g) ends up holding
//     O[head n][dims (D/4)·g .. (D/4)·g + D/4).
// The softmax state (max, sum) of head n lives in lanes n, n+16, n+32, n+48, so
// the rescale of O by exp(m_old − m_new) needs no cross-lane traffic.
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

template <int D>
struct PageRegs {
  uint4 k[D / 32];                      // K row (lane & 15), four 16-byte chunks per lane at D=128
  typename std::conditional<(D / 16) == 8, uint4, uint2>::type v[4];  // V rows 4g..4g+3
};

template <int D>
__device__ __forceinline__ void load_page(PageRegs<D>& r, const uint16_t* kbase, const uint16_t* vbase,
                                          const uint32_t (&koff)[D / 32], const uint32_t (&voff)[4]) {
#pragma unroll
  for (int c = 0; c < D / 32; ++c) r.k[c] = ld16(kbase + koff[c]);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (D / 16 == 8) r.v[j] = ld16(vbase + voff[j]);
    else r.v[j] = ld8(vbase + voff[j]);
  }
}

template <int D>
struct WaveState {
  float m;              // running max of head (lane & 15), log2 units
  float l;              // this lane's share of the running sum
  f32x4_t acc[D / 16];  // acc[c][i] = O[head][(D/16)·(4g+i) + c]
};

template <int D>
__device__ __forceinline__ void process_page(WaveState<D>& st, PageRegs<D>& r, const uint4 (&qb)[D / 32],
                                             int page, int seq_len, float scale_log2, int g) {
  constexpr int VD = D / 16;
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < D / 32; ++c) s = mfma_16x16x32(r.k[c], qb[c], s);

  const int tok0 = page * 16 + 4 * g;
  const bool partial = page * 16 + 16 > seq_len;  // wave-uniform
  float sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sv[i] = s[i] * scale_log2;
  if (partial) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (tok0 + i >= seq_len) sv[i] = kNegInf;
    }
    // Slots past seq_len may never have been written (NaN); P is 0 there, and
    // 0·NaN would poison the PV product, so the rows are zeroed.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (tok0 + j >= seq_len) {
        if constexpr (VD == 8) r.v[j] = make_uint4(0, 0, 0, 0);
        else r.v[j] = make_uint2(0, 0);
      }
    }
  }
  float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mx = max_across_groups(mx);
  const float m_new = fmaxf(st.m, mx);
  const float alpha = fast_exp2(st.m - m_new);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(sv[i] - m_new);
  st.l = st.l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  st.m = m_new;
#pragma unroll
  for (int c = 0; c < VD; ++c) st.acc[c] *= alpha;

  uint2 pb;
  pb.x = pack_bf16x2(p[0], p[1]);
  pb.y = pack_bf16x2(p[2], p[3]);
#pragma unroll
  for (int c = 0; c < VD; ++c) {
    uint2 va;
    if constexpr (VD == 8) {
      const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&r.v[0]);
      const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&r.v[1]);
      const uint32_t* v2 = reinterpret_cast<const uint32_t*>(&r.v[2]);
      const uint32_t* v3 = reinterpret_cast<const uint32_t*>(&r.v[3]);
      va.x = pick_halves(v0[c / 2], v1[c / 2], c & 1);
      va.y = pick_halves(v2[c / 2], v3[c / 2], c & 1);
    } else {
      const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&r.v[0]);
      const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&r.v[1]);
      const uint32_t* v2 = reinterpret_cast<const uint32_t*>(&r.v[2]);
      const uint32_t* v3 = reinterpret_cast<const uint32_t*>(&r.v[3]);
      va.x = pick_halves(v0[c / 2], v1[c / 2], c & 1);
      va.y = pick_halves(v2[c / 2], v3[c / 2], c & 1);
    }
    st.acc[c] = mfma_16x16x16(va, pb, st.acc[c]);
  }
}

template <int D, int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(DecodeArgs a) {
  constexpr int KC = D / 32;
  constexpr int VD = D / 16;
  constexpr int OD = D / 4;
  extern __shared__ float smem[];

  const int G = a.num_heads / a.num_kv_heads;
  const int wg = blockIdx.x;
  const int split = wg % a.num_splits;
  const int bk = wg / a.num_splits;
  const int kvh = bk % a.num_kv_heads;
  const int b = bk / a.num_kv_heads;

  const int lane = lane_id();
  const int n = lane & 15;
  const int g = lane >> 4;
  const int w = wave_id();

  const int seq_len = uniform(a.seq_lens[b]);
  int n_blocks = seq_len > 0 ? (seq_len + 15) / 16 : 0;
  n_blocks = min(n_blocks, a.max_blocks);
  const int start = split * a.blocks_per_split;
  const int end = (split == a.num_splits - 1) ? n_blocks : min(start + a.blocks_per_split, n_blocks);

  // Qᵀ operand: lane (n + 16g), chunk c -> q[b][kvh·G + n][8(4c+g) .. +8).
  uint4 qb[KC];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb +
                           (int64_t)(kvh * G + n) * a.q_sh;
#pragma unroll
    for (int c = 0; c < KC; ++c) qb[c] = (n < G) ? ld16(qrow + 8 * (4 * c + g)) : make_uint4(0, 0, 0, 0);
  }

  WaveState<D> st;
  st.m = kNegInf;
  st.l = 0.f;
#pragma unroll
  for (int c = 0; c < VD; ++c) st.acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t koff[KC], voff[4];
#pragma unroll
  for (int c = 0; c < KC; ++c) koff[c] = (uint32_t)(n * a.c_st + 8 * (4 * c + g));
#pragma unroll
  for (int j = 0; j < 4; ++j) voff[j] = (uint32_t)((4 * g + j) * a.c_st + VD * n);

  const uint16_t* kc = reinterpret_cast<const uint16_t*>(a.k_cache) + (int64_t)kvh * a.c_sh;
  const uint16_t* vc = reinterpret_cast<const uint16_t*>(a.v_cache) + (int64_t)kvh * a.c_sh;
  const int32_t* bt = a.block_tables + (int64_t)b * a.bt_stride;

  const int first = start + w;
  const int cnt = (end > first) ? (end - first + NW - 1) / NW : 0;
  for (int base = 0; base < cnt; base += 64) {
    const int here = min(64, cnt - base);
    // Lane k holds the table entry of this wave's page number base + k.
    int ent = 0;
    if (lane < here) ent = bt[first + NW * (base + lane)];
    ent = min(max(ent, 0), a.num_pages - 1);
    auto phys = [&](int k) -> int64_t { return (int64_t)__builtin_amdgcn_readlane(ent, k); };

    PageRegs<D> r0, r1;
    {
      const int64_t p0 = phys(0) * a.c_sb;
      load_page<D>(r0, kc + p0, vc + p0, koff, voff);
      const int64_t p1 = phys(min(1, here - 1)) * a.c_sb;
      load_page<D>(r1, kc + p1, vc + p1, koff, voff);
    }
    for (int k = 0; k < here; k += 2) {
      process_page<D>(st, r0, qb, first + NW * (base + k), seq_len, a.scale_log2, g);
      {
        const int64_t pn = phys(min(k + 2, here - 1)) * a.c_sb;
        load_page<D>(r0, kc + pn, vc + pn, koff, voff);
      }
      if (k + 1 < here) {
        process_page<D>(st, r1, qb, first + NW * (base + k + 1), seq_len, a.scale_log2, g);
        const int64_t pn = phys(min(k + 3, here - 1)) * a.c_sb;
        load_page<D>(r1, kc + pn, vc + pn, koff, voff);
      }
    }
  }
  const float l_tot = sum_across_groups(st.l);

  // Merge the NW wave states in wave order. LDS layout per wave:
  //   m[16], l[16], acc[G][D].
  const int wstride = 32 + G * D;
  float* my = smem + w * wstride;
  if (g == 0) {
    my[n] = st.m;
    my[16 + n] = l_tot;
  }
  if (n < G) {
    float* dst = my + 32 + n * D + OD * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int c = 0; c < VD; ++c) dst[VD * i + c] = st.acc[c][i];
    }
  }
  __syncthreads();

  const int total4 = G * D / 4;
  for (int e = threadIdx.x; e < total4; e += NW * 64) {
    const int h = (e * 4) / D;
    const int d = (e * 4) % D;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, smem[ww * wstride + h]);
    float L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    if (M != kNegInf) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float* ws = smem + ww * wstride;
        const float wgt = fast_exp2(ws[h] - M);
        L += ws[16 + h] * wgt;
        const float4 x = *reinterpret_cast<const float4*>(ws + 32 + h * D + d);
        A.x += x.x * wgt;
        A.y += x.y * wgt;
        A.z += x.z * wgt;
        A.w += x.w * wgt;
      }
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float4 o = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
    if (L == 0.f) o = make_float4(0.f, 0.f, 0.f, 0.f);
    const int head = kvh * G + h;
    if (a.num_splits == 1) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + d;
      uint2 pk;
      pk.x = pack_bf16x2(o.x, o.y);
      pk.y = pack_bf16x2(o.z, o.w);
      st8(dst, pk);
    } else {
      const int64_t row = ((int64_t)b * a.num_heads + head) * a.num_splits + split;
      *reinterpret_cast<float4*>(a.part_out + row * D + d) = o;
      if (d == 0) a.part_lse[row] = (L > 0.f) ? M + __log2f(L) : kNegInf;
    }
  }
}

// One work-group per (sequence, query head): out = Σ_s w_s·o_s / Σ_s w_s with
// w_s = 2^(lse_s − max lse). Thread (chunk, group) accumulates splits
// group, group + NG, ... in order, then the NG group sums are added in group
// order, so trailing empty splits (w = 0, o = 0) leave the bits unchanged.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeArgs a) {
  constexpr int CH = D / 4;       // float4 chunks per row
  constexpr int NG = 256 / CH;    // split groups
  __shared__ float red[256];
  __shared__ float4 gnum[NG][CH];
  __shared__ float gden[NG];

  const int bh = blockIdx.x;
  const int S = a.num_splits;
  const float* lse = a.part_lse + (int64_t)bh * S;
  const float* po = a.part_out + (int64_t)bh * S * D;

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
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + 4 * ch;
    uint2 pk;
    pk.x = pack_bf16x2(t.x * inv, t.y * inv);
    pk.y = pack_bf16x2(t.z * inv, t.w * inv);
    st8(dst, pk);
  }
}

template <int D, int NW>
static hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const int G = a.num_heads / a.num_kv_heads;
  const size_t smem = (size_t)NW * (32 + G * D) * sizeof(float);
  const int64_t wgs = (int64_t)a.batch * a.num_kv_heads * a.num_splits;
  if (wgs == 0) return hipSuccess;
  if (wgs > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_decode_kernel<D, NW>), dim3((unsigned)wgs), dim3(NW * 64), smem, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || a.num_splits == 1) return err;
  hipLaunchKernelGGL((decode_reduce_kernel<D>), dim3((unsigned)(a.batch * a.num_heads)), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

template <int D>
static hipError_t decode_for_dim(const DecodeArgs& a, hipStream_t stream) {
  switch (a.waves) {
    case 4: return launch_decode<D, 4>(a, stream);
    case 8: return launch_decode<D, 8>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t paged_decode(const DecodeArgs& a, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return decode_for_dim<64>(a, stream);
    case 128: return decode_for_dim<128>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
