// Kernel-bias chains of the disentangled attention (useCustomRelativeKernel,
// DeBERTa.swift:357-372): the relative-bias Metal kernel's bias
// fp16((c2p + p2c) * scale) with c2p, p2c in fp32 and masked keys := -65504
// (FusedKernels.swift:83-123), used as the whole SDPA mask (:383-385) or, on
// the explicit path, added to the fp16 content score with no where (:397-405).
// With the bias output this is gd_relative_bias on closed-form indices.
#include "deberta_attention_kernel.hpp"

namespace gd {

int launch_attention_kernel_bias(const AttentionArgs& a, hipStream_t stream) {
  if (a.score == kScoreKernelBiasExplicit) return launch_attention_sm<kScoreKernelBiasExplicit>(a, stream);
  return launch_attention_sm<kScoreKernelBias>(a, stream);
}

}  // namespace gd
