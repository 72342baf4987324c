// Fused residual add + RMSNorm, and SiLU(gate)·up: the two elementwise /
// row-reduction kernels of a decoder layer, both HBM-bound.
//
// fused_add_rms_norm replaces _fused_add_rms_norm_kernel
// (babyvllm/kernels/layernorm.py:5-83):
//   x = input (+ residual, rounded to bf16; the sum is written back to residual)
//   out = bf16( bf16(x · rsqrt(mean(x²) + eps)) · w )        (w bf16 or fp32)
// One wave per row: 16-byte loads, the row kept in registers between the sum
// of squares (fp32, wave reduction) and the scaling. Rows wider than the
// register budget, or not 16-byte aligned, take a two-pass scalar kernel.
//
// fused_silu_mul replaces _silu_mul_kernel (babyvllm/kernels/activation.py:5-65):
//   out[r, c] = bf16( silu(g) · u ),  g = gate_up[r, c], u = gate_up[r, D + c],
//   silu(g) = g · (1 / (1 + e^{-g})) in fp32 (hardware exp2 and reciprocal),
//   one rounding at the end.
#include "bvllm_device.h"
#include "bvllm_abi_internal.h"

namespace bvllm {

namespace {

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Round to bf16 with the hardware converter (v_cvt_pk_bf16_f32, round to
// nearest even), as a value and as packed pairs.
__device__ __forceinline__ float round_bf16(float x) { return lo_f32(pack_bf16x2_hw(x, 0.f)); }

__device__ __forceinline__ float add_bf16(float a, float b) { return round_bf16(a + b); }

__device__ __forceinline__ uint16_t norm_out(float x, float r, float w) {
  return (uint16_t)pack_bf16x2_hw(round_bf16(x * r) * w, 0.f);
}

template <bool W32>
__device__ __forceinline__ float weight_at(const void* w, int i) {
  if constexpr (W32) return reinterpret_cast<const float*>(w)[i];
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[i]);
}

// CPL: 16-byte chunks (8 bf16) per lane; the row has n ≤ 64·WPR·CPL·8
// elements. RPW rows per work-group with WPR waves per row (one of the two is
// 1): many rows take one wave each; a short batch (decode) splits each row
// over 4 waves, and the waves' sums of squares meet in LDS. The many-row form
// streams its input and residual with nontemporal loads (6% faster at 8192
// rows) and writes the sum and the output with nontemporal stores (5.1 ->
// 5.5 TB/s at 8192 rows); the short form keeps plain loads and stores, faster
// on the few rows the previous kernel has just written.
template <int CPL, bool HAS_RES, bool W32, int RPW, int WPR>
__global__ __launch_bounds__(64 * RPW * WPR) void rms_norm_vec_kernel(NormArgs a) {
  static_assert(RPW == 1 || WPR == 1, "rows per work-group or waves per row");
  __shared__ float wsum[RPW * WPR];
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.x * RPW + (RPW > 1 ? wave : 0);
  if (row >= a.rows) return;  // uniform over the work-group when WPR > 1
  const int lane = WPR > 1 ? (int)threadIdx.x : (int)(threadIdx.x & 63);  // lane within the row
  constexpr int LPR = 64 * WPR;                                             // lanes per row
  const int chunks = a.n / 8;
  const uint16_t* in = reinterpret_cast<const uint16_t*>(a.input) + (int64_t)row * a.in_stride;
  uint16_t* res = reinterpret_cast<uint16_t*>(a.residual) + (int64_t)row * a.res_stride;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.out_stride;

  // Row, residual and weight are all requested before the first use (one
  // memory round trip per row).
  uint4 xv[CPL];
  uint4 rv[CPL];
  uint4 wv[CPL][W32 ? 2 : 1];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + LPR * k;
    if constexpr (RPW > 1) {
      xv[k] = c < chunks ? ld16_nt(in + 8 * c) : make_uint4(0, 0, 0, 0);
      if (HAS_RES) rv[k] = c < chunks ? ld16_nt(res + 8 * c) : make_uint4(0, 0, 0, 0);
    } else {
      xv[k] = c < chunks ? ld16(in + 8 * c) : make_uint4(0, 0, 0, 0);
      if (HAS_RES) rv[k] = c < chunks ? ld16(res + 8 * c) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (W32) {
      const float* wp = reinterpret_cast<const float*>(a.weight) + 8 * c;
      wv[k][0] = c < chunks ? ld16(wp) : make_uint4(0, 0, 0, 0);
      wv[k][1] = c < chunks ? ld16(wp + 4) : make_uint4(0, 0, 0, 0);
    } else {
      wv[k][0] = c < chunks ? ld16(reinterpret_cast<const uint16_t*>(a.weight) + 8 * c) : make_uint4(0, 0, 0, 0);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    uint32_t* xw = reinterpret_cast<uint32_t*>(&xv[k]);
    if (HAS_RES) {
      const uint32_t* rw = reinterpret_cast<const uint32_t*>(&rv[k]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xw[q] = pack_bf16x2_hw(lo_f32(xw[q]) + lo_f32(rw[q]), hi_f32(xw[q]) + hi_f32(rw[q]));
      const int c = lane + LPR * k;
      if (c < chunks) {
        if constexpr (RPW > 1) st16_nt(res + 8 * c, xv[k]);
        else st16(res + 8 * c, xv[k]);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float l = lo_f32(xw[q]), h = hi_f32(xw[q]);
      ss = __builtin_fmaf(l, l, ss);
      ss = __builtin_fmaf(h, h, ss);
    }
  }
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    if ((threadIdx.x & 63) == 0) wsum[wave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < WPR; ++w) ss += wsum[w];
  }
  const float r = 1.f / sqrtf(ss / (float)a.n + a.eps);
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int c = lane + LPR * k;
    if (c >= chunks) continue;
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(&xv[k]);
    float w[8];
    if constexpr (W32) {
      const float* f0 = reinterpret_cast<const float*>(&wv[k][0]);
      const float* f1 = reinterpret_cast<const float*>(&wv[k][W32 ? 1 : 0]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        w[q] = f0[q];
        w[4 + q] = f1[q];
      }
    } else {
      const uint32_t* ww = reinterpret_cast<const uint32_t*>(&wv[k][0]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        w[2 * q] = lo_f32(ww[q]);
        w[2 * q + 1] = hi_f32(ww[q]);
      }
    }
    uint4 o;
    uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t n2 = pack_bf16x2_hw(lo_f32(xw[q]) * r, hi_f32(xw[q]) * r);  // bf16(x·r), two at a time
      ow[q] = pack_bf16x2_hw(lo_f32(n2) * w[2 * q], hi_f32(n2) * w[2 * q + 1]);
    }
    if constexpr (RPW > 1) st16_nt(out + 8 * c, o);
    else st16(out + 8 * c, o);
  }
}

// Any n and stride: one wave per row, two passes (the residual sum is written
// in the first and read back in the second).
template <bool HAS_RES, bool W32>
__global__ __launch_bounds__(256) void rms_norm_scalar_kernel(NormArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* in = reinterpret_cast<const uint16_t*>(a.input) + (int64_t)row * a.in_stride;
  uint16_t* res = reinterpret_cast<uint16_t*>(a.residual) + (int64_t)row * a.res_stride;
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + (int64_t)row * a.out_stride;
  float ss = 0.f;
  for (int i = lane; i < a.n; i += 64) {
    float x = bf16_to_f32(in[i]);
    if (HAS_RES) {
      x = add_bf16(x, bf16_to_f32(res[i]));
      res[i] = (uint16_t)f32_to_bf16_rne(x);
    }
    ss = __builtin_fmaf(x, x, ss);
  }
  ss = wave_sum(ss);
  const float r = 1.f / sqrtf(ss / (float)a.n + a.eps);
  const uint16_t* src = HAS_RES ? res : in;
  for (int i = lane; i < a.n; i += 64) out[i] = norm_out(bf16_to_f32(src[i]), r, weight_at<W32>(a.weight, i));
}

template <int CPL, int RPW, int WPR>
hipError_t launch_norm_vec_shape(const NormArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.rows + RPW - 1) / RPW)), block(64 * RPW * WPR);
  const bool res = a.residual != nullptr;
  if (res && a.weight_fp32)
    hipLaunchKernelGGL((rms_norm_vec_kernel<CPL, true, true, RPW, WPR>), grid, block, 0, s, a);
  else if (res)
    hipLaunchKernelGGL((rms_norm_vec_kernel<CPL, true, false, RPW, WPR>), grid, block, 0, s, a);
  else if (a.weight_fp32)
    hipLaunchKernelGGL((rms_norm_vec_kernel<CPL, false, true, RPW, WPR>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((rms_norm_vec_kernel<CPL, false, false, RPW, WPR>), grid, block, 0, s, a);
  return hipGetLastError();
}

// CPL is sized for one wave per row; with 4 waves per row each lane takes a
// quarter (rounded up).
template <int CPL>
hipError_t launch_norm_vec(const NormArgs& a, hipStream_t s) {
  if (a.rows >= 1024) return launch_norm_vec_shape<CPL, 4, 1>(a, s);
  return launch_norm_vec_shape<(CPL + 3) / 4, 1, 4>(a, s);
}

// sigmoid(g) = 1 / (1 + 2^(-g·log2 e)) with the hardware exp2 and reciprocal
// (about 1 ulp each in fp32, far below the final bf16 rounding) instead of the
// library expf and an IEEE division, which made the kernel VALU-bound.
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// Vector form: 8 gate and 8 up elements per thread, streamed with nontemporal
// loads and stores.
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                           int64_t total_chunks, int d_chunks) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total_chunks) return;
  const int64_t row = t / d_chunks;
  const int c = (int)(t - row * d_chunks);
  const uint16_t* g = gu + row * (int64_t)d_chunks * 16 + 8 * c;
  const uint4 gv = ld16_nt(g);
  const uint4 uv = ld16_nt(g + (int64_t)d_chunks * 8);
  const uint32_t* gw = reinterpret_cast<const uint32_t*>(&gv);
  const uint32_t* uw = reinterpret_cast<const uint32_t*>(&uv);
  uint4 o;
  uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float g0 = lo_f32(gw[q]), g1 = hi_f32(gw[q]);
    const float s0 = silu_f32(g0), s1 = silu_f32(g1);
    ow[q] = pack_bf16x2_hw(s0 * lo_f32(uw[q]), s1 * hi_f32(uw[q]));
  }
  st16_nt(out + row * (int64_t)d_chunks * 8 + 8 * c, o);
}

__global__ __launch_bounds__(256) void silu_mul_scalar_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                              int64_t total, int d) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int64_t row = t / d;
  const int c = (int)(t - row * d);
  const float g = bf16_to_f32(gu[row * 2 * d + c]);
  const float u = bf16_to_f32(gu[row * 2 * d + d + c]);
  out[t] = (uint16_t)f32_to_bf16_rne(silu_f32(g) * u);
}

}  // namespace

hipError_t fused_add_rms_norm(const NormArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.rows + 3) / 4));
  if (a.vec_ok) {
    const int chunks = a.n / 8;
    if (chunks <= 64 * 2) return launch_norm_vec<2>(a, s);
    if (chunks <= 64 * 4) return launch_norm_vec<4>(a, s);
    if (chunks <= 64 * 8) return launch_norm_vec<8>(a, s);
    if (chunks <= 64 * 16) return launch_norm_vec<16>(a, s);
  }
  const bool res = a.residual != nullptr;
  if (res && a.weight_fp32) hipLaunchKernelGGL((rms_norm_scalar_kernel<true, true>), grid, dim3(256), 0, s, a);
  else if (res) hipLaunchKernelGGL((rms_norm_scalar_kernel<true, false>), grid, dim3(256), 0, s, a);
  else if (a.weight_fp32) hipLaunchKernelGGL((rms_norm_scalar_kernel<false, true>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((rms_norm_scalar_kernel<false, false>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t silu_mul(const SiluArgs& a, hipStream_t s) {
  const uint16_t* gu = reinterpret_cast<const uint16_t*>(a.gate_up);
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
  if ((a.rows * a.d + 255) / 256 > 0x7fffffff) return hipErrorInvalidValue;
  if (a.vec_ok) {
    const int d_chunks = a.d / 8;
    const int64_t total = a.rows * d_chunks;
    hipLaunchKernelGGL(silu_mul_vec_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, gu, out, total,
                       d_chunks);
  } else {
    const int64_t total = a.rows * a.d;
    hipLaunchKernelGGL(silu_mul_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, gu, out,
                       total, a.d);
  }
  return hipGetLastError();
}

}  // namespace bvllm
