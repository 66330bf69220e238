// Alternative tile configurations of the forward grouped GEMM, selected at run time with
// MI355MOE_GG_VARIANT for measurement (the default configuration is gemm.hip's). They are compiled in
// their own translation unit so that the default kernels' code does not depend on them.
//   b6 - GGBig's 256 x 256 tiles with a sixth weight slot in the LDS of the MX weight row-scale ring
//        (bf16 and MX with EIO weights; MX with K-contiguous weights keeps the default).
//   dv - the direct-weight configuration of gemm_direct.hip (K-contiguous weights: bf16 EOI, MX EOI).
//   sp, sp4 - the split copy roles of gemm_split.hip (GEMMs on EIO weights, bf16 and MXFP8).
#include "gemm_kernel.h"

using GGB6 = GGCfg<256, 2, 3, 6, 1024, 1, 2, 0>;

int mi355_grouped_gemm_variant(const GGParams& p, bool mx, bool b_kn, int epi, hipStream_t stream, int variant) {
  if (variant == MI355_GG_VARIANT_B6) return dispatch_gg<GGB6>(p, mx, b_kn, epi, stream);
  if (variant == MI355_GG_VARIANT_DV && mi355_direct_gemm_enabled()) return mi355_grouped_gemm_direct(p, mx, b_kn, epi, stream);
  if ((variant == MI355_GG_VARIANT_SP || variant == MI355_GG_VARIANT_SP4) && mi355_split_roles_enabled())
    return mi355_grouped_gemm_split(p, mx, b_kn, epi, stream, variant);
  return MI355MOE_EUNSUPPORTED;
}
