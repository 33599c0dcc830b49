// Explicit-score chain of the disentangled attention (useFastAttention =
// false, DeBERTa.swift:397-409): fp16(fp16(q.k) / fp16(sqrt(3D))) plus the
// default graph's fp16 bias in fp16, masked keys excluded, fp16
// probabilities, fp16(P.V).
#include "deberta_attention_kernel.hpp"

namespace gd {

int launch_attention_explicit(const AttentionArgs& a, hipStream_t stream) {
  return launch_attention_sm<kScoreExplicit>(a, stream);
}

}  // namespace gd
