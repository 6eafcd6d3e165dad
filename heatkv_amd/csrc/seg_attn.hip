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
// The append after a kernel that does not fuse it (AttnArgs::append_offsets).
__global__ __launch_bounds__(256) void append_kernel(const AttnArgs a, int32_t k_row, int32_t v_row) {
  attn::append_block<256>(a, blockIdx.x, k_row, v_row);
}

hipError_t launch_append(const AttnArgs& a, hipStream_t stream) {
  const int64_t blocks = attn::append_blocks(a.batch, a.heads, a.cur_len);
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  // split rows and fp32 rows are 4 bytes per element, 16-bit rows 2
  const int32_t k_row = (a.k_dtype == kSplitRows || a.k_dtype == kF32 ? 4 : 2) * attn::kD;
  const int32_t v_row = (a.v_dtype == kF32 ? 4 : 2) * attn::kD;
  append_kernel<<<dim3(static_cast<uint32_t>(blocks)), 256, 0, stream>>>(a, k_row, v_row);
  return hipGetLastError();
}

bool force_staged() {
  static const bool v = [] {
    const char* e = std::getenv("HKV_ATTN_PATH");
    return e != nullptr && std::strcmp(e, "staged") == 0;
  }();
  return v;
}
}  // namespace

int32_t attention_workgroups_per_cu(const AttnArgs& a) {
  if (a.k_dtype == kSplitRows) return 1;
  if (!force_staged() && attention_direct_supported(a)) return 2;
  // the staged kernel's split modes (3-piece q/k, fp32 value mode, fp32 V)
  // hold more pieces per wave: one workgroup per CU
  const bool split = (a.q_dtype == kF32 && a.qk_dot_mode == kDotFp32) || a.value_dot_mode == kDotFp32 ||
                     a.v_dtype == kF32;
  return split ? 1 : 2;
}

hipError_t launch_segmented_attention(const AttnArgs& a, hipStream_t stream) {
  if (a.heads > attn::kMaxHeads) return hipErrorInvalidValue;
  attn::Scalars s;
  const float scale_abs = a.softmax_scale < 0.f ? -a.softmax_scale : a.softmax_scale;
  s.c = fmaxf(scale_abs * attn::kLog2e, attn::kMinC);
  s.thresh = attn::kRescaleLog2 / s.c;
  s.q_sign = a.softmax_scale < 0.f ? 0x80008000u : 0u;
  hipError_t e;
  if (a.k_dtype == kSplitRows) {
    e = launch_attention_split(a, s, stream);
  } else {
    if (a.q_dtype != a.k_dtype) return hipErrorInvalidValue;
    // the 16-bit kernel runs the append in its own launch
    if (!force_staged() && attention_direct_supported(a)) return launch_attention_direct(a, s, stream);
    e = launch_attention_staged(a, s, stream);
  }
  if (e != hipSuccess || a.append_offsets == nullptr) return e;
  return launch_append(a, stream);
}

}  // namespace hkv
