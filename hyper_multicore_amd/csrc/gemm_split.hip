// Split copy roles (variants sp / sp4) of the forward grouped GEMM: waves 0-1 copy the activations,
// waves 2-3 the weights, so each wave's in-order load counter covers one stream and the weight ring
// hides HBM latency with its full depth (GGCfg::SPLIT, gemm_plan.h). GEMMs on EIO weights: the
// reference's MXFP8 roots (col_data / col_scale) and bf16 [E, K, N]; K-contiguous weights have the
// direct-weight configuration. Own translation unit, so the default kernels' code does not depend on
// these.
//   sp  - 3 activation and 6 weight slots
//   sp4 - 4 activation and 5 weight slots
#include "gemm_kernel.h"

using GGSplit = GGCfg<256, 2, 3, 6, 1024, 1, 2, 0, true>;
using GGSplitA4 = GGCfg<256, 2, 4, 5, 1024, 1, 2, 0, true>;

template <class C>
static int dispatch_split(const GGParams& p, bool mx, int epi, hipStream_t stream) {
  if (mx) {
    if (epi == EPI_SWIGLU_MX) return launch_gg<C, true, true, EPI_SWIGLU_MX>(p, stream);
    return launch_gg<C, true, true, EPI_STORE_BF16>(p, stream);
  }
  if (epi == EPI_SWIGLU_BF16) return launch_gg<C, false, true, EPI_SWIGLU_BF16>(p, stream);
  return launch_gg<C, false, true, EPI_STORE_BF16>(p, stream);
}

int mi355_grouped_gemm_split(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, int variant) {
  if (!gg_split_applies(p, mx, b_kn, epi)) return MI355MOE_EUNSUPPORTED;
  if (variant == MI355_GG_VARIANT_SP) return dispatch_split<GGSplit>(p, mx, epi, stream);
  if (variant == MI355_GG_VARIANT_SP4) return dispatch_split<GGSplitA4>(p, mx, epi, stream);
  return MI355MOE_EUNSUPPORTED;
}
