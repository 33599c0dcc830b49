// Default score chain of the disentangled attention: the default graph's
// fp16 relative bias and SDPA with bias + key mask (DeBERTa.swift:374-394).
#include "deberta_attention_kernel.hpp"

namespace gd {

int launch_attention_default(const AttentionArgs& a, hipStream_t stream) {
  return launch_attention_sm<kScoreDefault>(a, stream);
}

}  // namespace gd
