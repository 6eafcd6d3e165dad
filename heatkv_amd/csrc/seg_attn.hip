// Segmented attention launch: the split-row kernel for K in split rows
// (seg_attn_split.hip), the direct-to-LDS kernel for 16-bit K/V
// (seg_attn_direct.hip) and the register-staged kernel otherwise
// (seg_attn_staged.hip).  HKV_ATTN_PATH=staged (read once) forces the staged
// kernel, for comparisons.
#include <cstdlib>
#include <cstring>

#include "attn_common.h"

namespace hkv {

namespace {
bool force_staged() {
  static const bool v = [] {
    const char* e = std::getenv("HKV_ATTN_PATH");
    return e != nullptr && std::strcmp(e, "staged") == 0;
  }();
  return v;
}
}  // namespace

hipError_t launch_segmented_attention(const AttnArgs& a, hipStream_t stream) {
  if (a.heads > attn::kMaxHeads) return hipErrorInvalidValue;
  attn::Scalars s;
  const float scale_abs = a.softmax_scale < 0.f ? -a.softmax_scale : a.softmax_scale;
  s.c = fmaxf(scale_abs * attn::kLog2e, attn::kMinC);
  s.thresh = attn::kRescaleLog2 / s.c;
  s.q_sign = a.softmax_scale < 0.f ? 0x80008000u : 0u;
  if (a.k_dtype == kSplitRows) return launch_attention_split(a, s, stream);
  if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
  if (!force_staged() && attention_direct_supported(a)) return launch_attention_direct(a, s, stream);
  return launch_attention_staged(a, s, stream);
}

}  // namespace hkv
