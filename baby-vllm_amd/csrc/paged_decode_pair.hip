// Two-wave split decode for the plans whose pair kernels run faster with the
// MFMA accumulators in VGPRs: the group walks (one work-group per group of
// splits; the split merges then copy no accumulator between AGPRs and VGPRs)
// and the D = 64 split walk. build_lib.py compiles this file with
// -mllvm -amdgpu-mfma-vgpr-form. Measured against the same kernels built with
// AGPR accumulators: B1 x 32768 (group walk) 20.85 -> 20.55 us, config 1
// (D = 64 split walk) 11.28 -> 11.13 us; the D = 128 split walk (B8 x 1920)
// ran 14.38 -> 14.57 us that way and stays in paged_decode.hip. The four-wave
// split walk at D = 64 lives here too (config 1 10.76 -> 10.68 us).
#include "paged_decode_stream.h"

namespace bvllm {

template <int D>
static hipError_t launch_pair_dim(const DecodeArgs& a, int64_t items, bool group, bool nt, hipStream_t stream) {
  const dim3 grid((unsigned)items), block(128);
  if (group && nt) hipLaunchKernelGGL((paged_decode_pair_kernel<D, true, true>), grid, block, 0, stream, a, (int)items);
  else if (group) hipLaunchKernelGGL((paged_decode_pair_kernel<D, false, true>), grid, block, 0, stream, a, (int)items);
  else if constexpr (D == 64) {
    if (nt) hipLaunchKernelGGL((paged_decode_pair_kernel<D, true, false>), grid, block, 0, stream, a, (int)items);
    else hipLaunchKernelGGL((paged_decode_pair_kernel<D, false, false>), grid, block, 0, stream, a, (int)items);
  } else {
    return hipErrorInvalidValue;  // D = 128 split walks launch from paged_decode.hip
  }
  return hipGetLastError();
}

hipError_t launch_pair_vgpr(const DecodeArgs& a, int64_t items, bool group, bool nt, hipStream_t stream) {
  switch (a.head_dim) {
    case 64: return launch_pair_dim<64>(a, items, group, nt, stream);
    case 128: return launch_pair_dim<128>(a, items, group, nt, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_quad_vgpr(const DecodeArgs& a, int64_t items, bool nt, hipStream_t stream) {
  switch (a.head_dim) {
    case 64:
      if (nt) hipLaunchKernelGGL((paged_decode_quad_kernel<64, true>), dim3((unsigned)items), dim3(256), 0, stream, a, (int)items);
      else hipLaunchKernelGGL((paged_decode_quad_kernel<64, false>), dim3((unsigned)items), dim3(256), 0, stream, a, (int)items);
      return hipGetLastError();
    default: return hipErrorInvalidValue;  // D = 128 launches from paged_decode.hip
  }
}

}  // namespace bvllm
