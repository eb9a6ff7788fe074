// Variable batch size per feature ("VBE") metadata for gfx950.
//
// Semantics: fbgemm_gpu generate_vbe_metadata (upstream
// src/split_embeddings_utils/, recalled).  Features (tables) t have their own
// batch, split over R ranks: rank r holds B[t][r] samples of feature t.  The
// flattened bag space is feature-major, and within a feature rank-major:
//   bag(t, b) = B_offsets[t] + b,   b = B_offsets_rank_per_feature[t][r] + b_r.
// The pooled output is one flat buffer, rank-major then feature-major: the
// block of (rank r, feature t) starts at output_offsets_feature_rank[r*T + t]
// and holds B[t][r] rows of D_t (or of a fixed D for sequence lookups).
// Per bag this kernel writes
//   row_output_offsets[bag] = output_offsets_feature_rank[r*T + t] + b_r * D_t
//   b_t_map[bag]            = (t << info_B_num_bits) | b.
// One thread per bag: the feature by a binary search over B_offsets, the rank
// by one over that feature's rank offsets (both tiny, cached).
#include "mx_common.h"

namespace mx {
namespace {

__global__ void __launch_bounds__(256)
    vbe_metadata_kernel(const int32_t* __restrict__ B_offsets,
                        const int32_t* __restrict__ B_offsets_rpf,
                        const int64_t* __restrict__ out_offsets_fr,
                        const int32_t* __restrict__ D_offsets, int32_t fixed_D, int32_t T,
                        int32_t R, int32_t nb, int64_t total_B,
                        int64_t* __restrict__ row_out, int32_t* __restrict__ b_t_map) {
  const int64_t bag = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (bag >= total_B) return;
  int32_t lo = 0, hi = T;  // B_offsets[lo] <= bag < B_offsets[hi]
  while (hi - lo > 1) {
    const int32_t mid = lo + ((hi - lo) >> 1);
    if (B_offsets[mid] <= bag)
      lo = mid;
    else
      hi = mid;
  }
  const int32_t t = lo;
  const int64_t b = bag - B_offsets[t];
  const int32_t* rpf = B_offsets_rpf + static_cast<int64_t>(t) * (R + 1);
  int32_t rlo = 0, rhi = R;  // rpf[rlo] <= b < rpf[rhi]
  while (rhi - rlo > 1) {
    const int32_t mid = rlo + ((rhi - rlo) >> 1);
    if (rpf[mid] <= b)
      rlo = mid;
    else
      rhi = mid;
  }
  const int64_t b_r = b - rpf[rlo];
  const int64_t D = fixed_D > 0 ? fixed_D : D_offsets[t + 1] - D_offsets[t];
  row_out[bag] = out_offsets_fr[static_cast<int64_t>(rlo) * T + t] + b_r * D;
  b_t_map[bag] = static_cast<int32_t>((nb >= 32 ? 0u : (static_cast<uint32_t>(t) << nb)) |
                                      static_cast<uint32_t>(b));
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_generate_vbe_metadata(const int32_t* B_offsets,
                                        const int32_t* B_offsets_rank_per_feature,
                                        const int64_t* output_offsets_feature_rank,
                                        const int32_t* D_offsets, int32_t fixed_D, int32_t T,
                                        int32_t R, int32_t info_B_num_bits, int64_t total_B,
                                        int64_t* row_output_offsets, int32_t* b_t_map,
                                        void* stream) {
  clear_error();
  MX_REQUIRE(T >= 1 && R >= 1 && total_B >= 0, "T=%d, R=%d, total_B=%lld invalid", T, R,
             (long long)total_B);
  MX_REQUIRE(info_B_num_bits >= 1 && info_B_num_bits <= 32, "info_B_num_bits %d invalid",
             info_B_num_bits);
  MX_REQUIRE(fixed_D >= 0, "negative D");
  if (total_B == 0) return MX_OK;
  MX_REQUIRE(B_offsets && B_offsets_rank_per_feature && output_offsets_feature_rank &&
                 (fixed_D > 0 || D_offsets) && row_output_offsets && b_t_map,
             "null pointer argument");
  vbe_metadata_kernel<<<dim3(static_cast<uint32_t>(ceil_div(total_B, 256))), 256, 0,
                        as_stream(stream)>>>(B_offsets, B_offsets_rank_per_feature,
                                             output_offsets_feature_rank, D_offsets, fixed_D, T, R,
                                             info_B_num_bits, total_B, row_output_offsets,
                                             b_t_map);
  MX_LAUNCH_CHECK();
  return MX_OK;
}
