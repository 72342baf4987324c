// Fused rotate-half RoPE on q and k (in place) + scatter of rotated k and raw v
// into the paged KV cache through slot_mapping.
//
// Replaces the reference's _rope_kv_cache_kernel (babyvllm/kernels/rope.py:5-98).
//
// Work decomposition: one thread per "item" of a token, items laid out so that
// consecutive threads touch consecutive 16-byte chunks of the same head rows:
//   * rotation items: (head in q heads ++ k heads, chunk c of the first half);
//     a thread loads x1 = x[c·VW .. +VW) and x2 = x[D/2 + c·VW .. +VW), the
//     matching cos/sin chunks, and writes both halves back (and, for k heads,
//     also into the cache row of the token's slot);
//   * copy items (only with a cache): (kv head, chunk of D) of v -> v_cache.
// All loads/stores are VW-wide (8 bf16 = 16 B when aligned), so every wave
// reads whole 128-byte lines of the token's q/k/v rows.
//
// Rounding follows torch's eager bf16 elementwise ops: each product rounds to
// bf16, then the sum rounds to bf16 (no fused multiply-add).
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
