// Fused chain of the disentangled attention (useFusedAttentionKernel,
// DeBERTa.swift:337-354): the fused Metal kernel's score
// (q.k + c2p + p2c) * scale in fp32, masked keys excluded, softmax and P.V
// (FusedKernels.swift:13-81); gd_fused_attention on closed-form indices.
#include "deberta_attention_kernel.hpp"

namespace gd {

int launch_attention_fused(const AttentionArgs& a, hipStream_t stream) {
  return launch_attention_sm<kScoreFused>(a, stream);
}

}  // namespace gd
