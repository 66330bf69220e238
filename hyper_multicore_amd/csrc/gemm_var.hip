// Alternative tile configurations of the forward grouped GEMM, selected at run time with
// MI355MOE_GG_VARIANT for measurement (the default configuration is gemm.hip's). They are compiled in
// their own translation unit so that the default kernels' code does not depend on them.
//   b6 - GGBig's 256 x 256 tiles with a sixth weight slot in the LDS of the MX weight row-scale ring
//        (bf16 and MX with EIO weights; MX with K-contiguous weights keeps the default).
//   dv - the direct-weight configuration of gemm_direct.hip (K-contiguous weights: bf16 EOI, MX EOI).
//   sp - split copy roles (waves 0-1 copy activations, 2-3 weights) with 3 activation and 6 weight
//        slots; sp4 - the same with 4 and 5 (MXFP8 GEMMs on EIO weight roots).
#include "gemm_kernel.h"

using GGB6 = GGCfg<256, 2, 3, 6, 1024, 1, 2, 0>;
using GGSplit = GGCfg<256, 2, 3, 6, 1024, 1, 2, 0, true>;
using GGSplitA4 = GGCfg<256, 2, 4, 5, 1024, 1, 2, 0, true>;

template <class C>
static int dispatch_split(const GGParams& p, int epi, hipStream_t stream) {
  if (epi == EPI_SWIGLU_MX) return launch_gg<C, true, true, EPI_SWIGLU_MX>(p, stream);
  return launch_gg<C, true, true, EPI_STORE_BF16>(p, stream);
}

int mi355_grouped_gemm_variant(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, int variant) {
  if (variant == MI355_GG_VARIANT_B6) return dispatch_gg<GGB6>(p, mx, b_kn, epi, stream);
  if (variant == MI355_GG_VARIANT_DV && mi355_direct_gemm_enabled()) return mi355_grouped_gemm_direct(p, mx, b_kn, epi, stream);
  // split roles: MXFP8 with the reference's EIO weight roots (bf16 EOI has the direct configuration)
  if (gg_split_applies(p, mx, b_kn, epi)) {
    if (variant == MI355_GG_VARIANT_SP && mi355_split_roles_enabled()) return dispatch_split<GGSplit>(p, epi, stream);
    if (variant == MI355_GG_VARIANT_SP4 && mi355_split_roles_enabled()) return dispatch_split<GGSplitA4>(p, epi, stream);
  }
  return MI355MOE_EUNSUPPORTED;
}
