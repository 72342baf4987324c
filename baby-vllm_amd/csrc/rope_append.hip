// Fused rotate-half RoPE on q and k (in place) + scatter of rotated k and raw v
// into the paged KV cache through slot_mapping.
//
// Replaces the reference's _rope_kv_cache_kernel (babyvllm/kernels/rope.py:5-98).
//
// Two kernels with the same results:
//   * the row kernel (below: rope_append_rows_kernel), used whenever every row
//     start and stride is 16-byte aligned: each wave moves whole head rows of
//     one token in 16-byte chunks, with streaming (nontemporal) loads and stores;
//   * the chunk kernel (rope_kv_append_kernel), for any alignment: one thread
//     per "item" of a token, items laid out so that consecutive threads touch
//     consecutive VW-element chunks of the same head rows —
//       rotation items: (head in q heads ++ k heads, chunk c of the first half);
//       a thread loads x1 = x[c·VW .. +VW) and x2 = x[D/2 + c·VW .. +VW), the
//       matching cos/sin chunks, and writes both halves back (and, for k heads,
//       also into the cache row of the token's slot);
//       copy items (only with a cache): (kv head, chunk of D) of v -> v_cache.
//
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

template <int VW>
struct Chunk {
  uint16_t h[VW];
};

// NT: the data is read once per call (q, k, v rows), loaded with the
// nontemporal hint; cos/sin rows are shared by all heads of a token.
template <int VW, bool NT = false>
__device__ __forceinline__ Chunk<VW> load_chunk(const uint16_t* p) {
  Chunk<VW> c;
  if constexpr (VW == 8) {
    uint4 v = NT ? ld16_nt(p) : ld16(p);
    c = __builtin_bit_cast(Chunk<VW>, v);
  } else if constexpr (VW == 4) {
    uint2 v = ld8(p);
    c = __builtin_bit_cast(Chunk<VW>, v);
  } else {
#pragma unroll
    for (int i = 0; i < VW; ++i) c.h[i] = p[i];
  }
  return c;
}

template <int VW>
__device__ __forceinline__ void store_chunk(uint16_t* p, const Chunk<VW>& c) {
  if constexpr (VW == 8) {
    st16(p, __builtin_bit_cast(uint4, c));
  } else if constexpr (VW == 4) {
    st8(p, __builtin_bit_cast(uint2, c));
  } else {
#pragma unroll
    for (int i = 0; i < VW; ++i) p[i] = c.h[i];
  }
}

// o1 = bf16(bf16(x1·c1) − bf16(x2·s1)),  o2 = bf16(bf16(x2·c2) + bf16(x1·s2))
template <int VW>
__device__ __forceinline__ void rotate(Chunk<VW>& x1, Chunk<VW>& x2, const Chunk<VW>& c1,
                                       const Chunk<VW>& c2, const Chunk<VW>& s1,
                                       const Chunk<VW>& s2) {
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const float a = bf16_to_f32(x1.h[i]);
    const float b = bf16_to_f32(x2.h[i]);
    const float a_c = bf16_to_f32(f32_to_bf16_rne(a * bf16_to_f32(c1.h[i])));
    const float b_s = bf16_to_f32(f32_to_bf16_rne(b * bf16_to_f32(s1.h[i])));
    const float b_c = bf16_to_f32(f32_to_bf16_rne(b * bf16_to_f32(c2.h[i])));
    const float a_s = bf16_to_f32(f32_to_bf16_rne(a * bf16_to_f32(s2.h[i])));
    x1.h[i] = (uint16_t)f32_to_bf16_rne(a_c - b_s);
    x2.h[i] = (uint16_t)f32_to_bf16_rne(b_c + a_s);
  }
}

template <int D, int VW>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(RopeArgs a) {
  constexpr int HALF = D / 2;
  constexpr int RC = HALF / VW;  // rotation chunks per head
  constexpr int VC = D / VW;     // copy chunks per v head
  const int rot_items = (a.num_heads + a.num_kv_heads) * RC;
  const int items = rot_items + (a.has_cache ? a.num_kv_heads * VC : 0);
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.num_tokens * items;
  if (gid >= total) return;
  const int t = (int)(gid / items);
  const int it = (int)(gid - (int64_t)t * items);

  uint16_t* qp = reinterpret_cast<uint16_t*>(a.q);
  uint16_t* kp = reinterpret_cast<uint16_t*>(a.k);
  const uint16_t* vp = reinterpret_cast<const uint16_t*>(a.v);

  int64_t slot = -1;
  if (a.has_cache) {
    slot = a.slot_mapping[t];
    if (slot < 0 || slot >= a.num_slots) slot = -1;  // out-of-range slots are not written
  }

  if (it < rot_items) {
    const int head = it / RC;
    const int c = it - head * RC;
    const bool is_k = head >= a.num_heads;
    const int hk = head - a.num_heads;
    uint16_t* row = is_k ? kp + (int64_t)t * a.k_st + (int64_t)hk * a.k_sh
                         : qp + (int64_t)t * a.q_st + (int64_t)head * a.q_sh;
    const uint16_t* cs = reinterpret_cast<const uint16_t*>(a.cos) + (int64_t)t * a.cs_st;
    const uint16_t* sn = reinterpret_cast<const uint16_t*>(a.sin) + (int64_t)t * a.sn_st;
    Chunk<VW> x1 = load_chunk<VW, true>(row + c * VW);
    Chunk<VW> x2 = load_chunk<VW, true>(row + HALF + c * VW);
    const Chunk<VW> c1 = load_chunk<VW>(cs + c * VW);
    const Chunk<VW> c2 = load_chunk<VW>(cs + HALF + c * VW);
    const Chunk<VW> s1 = load_chunk<VW>(sn + c * VW);
    const Chunk<VW> s2 = load_chunk<VW>(sn + HALF + c * VW);
    rotate<VW>(x1, x2, c1, c2, s1, s2);
    store_chunk<VW>(row + c * VW, x1);
    store_chunk<VW>(row + HALF + c * VW, x2);
    if (is_k && slot >= 0) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.k_cache) + slot * a.kc_slot + (int64_t)hk * a.kc_head;
      store_chunk<VW>(dst + c * VW, x1);
      store_chunk<VW>(dst + HALF + c * VW, x2);
    }
  } else {
    const int j = it - rot_items;
    const int hv = j / VC;
    const int c = j - hv * VC;
    if (slot >= 0) {
      const uint16_t* src = vp + (int64_t)t * a.v_st + (int64_t)hv * a.v_sh;
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.v_cache) + slot * a.vc_slot + (int64_t)hv * a.vc_head;
      store_chunk<VW>(dst + c * VW, load_chunk<VW, true>(src + c * VW));
    }
  }
}

// Row kernel: one wave-wide pass ("unit") per wave.
//
// A token's work is cut into units: a rotation unit covers RPI = 64 / (D/16)
// q or k head rows (lane = (row, chunk c of the first half); the lane loads
// x1 = row[c·8 .. +8) and x2 = row[D/2 + c·8 .. +8) and the token's matching
// cos/sin chunks), a copy unit covers 64 / (D/8) v head rows. At the 7B shape
// a token is 5 units (32 rotated rows in 4, 4 v rows in 1), so 5 waves. The
// rows are read with the nontemporal hint and written with it (q, k in place
// and both cache rows), which measured 1.3x the rate of plain stores here; one
// unit per wave beat 2, 4 or all 5 units per wave (fewer waves in flight).
// Products and sums round to bf16 with the hardware converter (round to nearest
// even: the same bits as the software rounding for every non-NaN value; a NaN
// stays NaN, its sign and payload unspecified).
__device__ __forceinline__ void rotate_hw(uint4& x1, uint4& x2, const float* c1, const float* c2,
                                          const float* s1, const float* s2) {
  uint32_t w1[4] = {x1.x, x1.y, x1.z, x1.w}, w2[4] = {x2.x, x2.y, x2.z, x2.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a0 = lo_f32(w1[i]), a1 = hi_f32(w1[i]);
    const float b0 = lo_f32(w2[i]), b1 = hi_f32(w2[i]);
    const uint32_t ac = pack_bf16x2_hw(a0 * c1[2 * i], a1 * c1[2 * i + 1]);
    const uint32_t bs = pack_bf16x2_hw(b0 * s1[2 * i], b1 * s1[2 * i + 1]);
    const uint32_t bc = pack_bf16x2_hw(b0 * c2[2 * i], b1 * c2[2 * i + 1]);
    const uint32_t as = pack_bf16x2_hw(a0 * s2[2 * i], a1 * s2[2 * i + 1]);
    w1[i] = pack_bf16x2_hw(lo_f32(ac) - lo_f32(bs), hi_f32(ac) - hi_f32(bs));
    w2[i] = pack_bf16x2_hw(lo_f32(bc) + lo_f32(as), hi_f32(bc) + hi_f32(as));
  }
  x1 = make_uint4(w1[0], w1[1], w1[2], w1[3]);
  x2 = make_uint4(w2[0], w2[1], w2[2], w2[3]);
}

__device__ __forceinline__ void to_floats(const uint4& c, float* f) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo_f32(w[i]);
    f[2 * i + 1] = hi_f32(w[i]);
  }
}

template <int D>
__global__ __launch_bounds__(256) void rope_append_rows_kernel(RopeArgs a, int32_t units) {
  constexpr int HALF = D / 2;
  constexpr int RC = HALF / 8, RPI = 64 / RC;  // lanes per rotated row, rows per rotation unit
  constexpr int VC = D / 8, VPI = 64 / VC;     // lanes per v row, rows per copy unit
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x / 64) + wave_id();
  const int64_t t64 = wave / units;
  if (t64 >= a.num_tokens) return;
  const int t = (int)t64;
  const int u = (int)(wave - t64 * units);
  const int lane = lane_id();
  const int rows = a.num_heads + a.num_kv_heads;
  const int rot_units = (rows + RPI - 1) / RPI;

  int64_t slot = -1;
  if (a.has_cache) {
    slot = a.slot_mapping[t];
    if (slot < 0 || slot >= a.num_slots) slot = -1;  // out-of-range slots are not written
  }
  if (u >= rot_units) {  // copy unit: v rows into the cache
    const int hv = (u - rot_units) * VPI + lane / VC;
    const int c = lane % VC;
    if (hv < a.num_kv_heads && slot >= 0) {
      const uint16_t* src = reinterpret_cast<const uint16_t*>(a.v) + (int64_t)t * a.v_st + (int64_t)hv * a.v_sh;
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.v_cache) + slot * a.vc_slot + (int64_t)hv * a.vc_head;
      st16_nt(dst + c * 8, ld16_nt(src + c * 8));
    }
    return;
  }
  const int c = lane % RC;
  const int row = u * RPI + lane / RC;
  if (row >= rows) return;
  const bool is_k = row >= a.num_heads;
  const int hk = row - a.num_heads;
  uint16_t* p = is_k ? reinterpret_cast<uint16_t*>(a.k) + (int64_t)t * a.k_st + (int64_t)hk * a.k_sh
                     : reinterpret_cast<uint16_t*>(a.q) + (int64_t)t * a.q_st + (int64_t)row * a.q_sh;
  uint4 x1 = ld16_nt(p + c * 8);
  uint4 x2 = ld16_nt(p + HALF + c * 8);
  const uint16_t* cs = reinterpret_cast<const uint16_t*>(a.cos) + (int64_t)t * a.cs_st + c * 8;
  const uint16_t* sn = reinterpret_cast<const uint16_t*>(a.sin) + (int64_t)t * a.sn_st + c * 8;
  float c1[8], c2[8], s1[8], s2[8];
  to_floats(ld16(cs), c1);
  to_floats(ld16(cs + HALF), c2);
  to_floats(ld16(sn), s1);
  to_floats(ld16(sn + HALF), s2);
  rotate_hw(x1, x2, c1, c2, s1, s2);
  st16_nt(p + c * 8, x1);
  st16_nt(p + HALF + c * 8, x2);
  if (is_k && slot >= 0) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(a.k_cache) + slot * a.kc_slot + (int64_t)hk * a.kc_head + c * 8;
    st16_nt(dst, x1);
    st16_nt(dst + HALF, x2);
  }
}

template <int D>
static hipError_t launch_rows(const RopeArgs& a, hipStream_t stream) {
  constexpr int RPI = 64 / (D / 16), VPI = 64 / (D / 8);
  const int units = (a.num_heads + a.num_kv_heads + RPI - 1) / RPI +
                    (a.has_cache ? (a.num_kv_heads + VPI - 1) / VPI : 0);
  const int64_t waves = (int64_t)a.num_tokens * units;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((rope_append_rows_kernel<D>), dim3((unsigned)blocks), dim3(256), 0, stream, a, units);
  return hipGetLastError();
}

template <int D, int VW>
static hipError_t launch_rope(const RopeArgs& a, hipStream_t stream) {
  const int rc = (D / 2) / VW, vc = D / VW;
  const int64_t items = (int64_t)(a.num_heads + a.num_kv_heads) * rc +
                        (a.has_cache ? (int64_t)a.num_kv_heads * vc : 0);
  const int64_t total = items * a.num_tokens;
  const int64_t blocks = (total + 255) / 256;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((rope_kv_append_kernel<D, VW>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t rope_kv_append(const RopeArgs& a, hipStream_t stream) {
  if (a.vec_ok && tuning(kTuneAppendChunks) == 0) {
    switch (a.head_dim) {
      case 64: return launch_rows<64>(a, stream);
      case 128: return launch_rows<128>(a, stream);
      case 256: return launch_rows<256>(a, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (a.head_dim) {
    case 64:
      return a.vec_ok ? launch_rope<64, 8>(a, stream) : launch_rope<64, 1>(a, stream);
    case 128:
      return a.vec_ok ? launch_rope<128, 8>(a, stream) : launch_rope<128, 1>(a, stream);
    case 256:
      return a.vec_ok ? launch_rope<256, 8>(a, stream) : launch_rope<256, 1>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace bvllm
