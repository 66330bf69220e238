// Feature gates of the optional paths (reported by mi355moe_features).
#pragma once
#include <stdlib.h>
#include <string.h>

// Optional paths. Each was switched on after its GPU parity tests passed; a path switched off answers
// MI355MOE_EUNSUPPORTED (or the forward keeps the default tiles) and mi355moe_features() clears its
// bit, which the GPU tests of that path read to skip.
// MX GEMM with K-contiguous (EOI) weights.
inline bool mi355_mx_eoi_enabled() { return true; }
// BF16 numerics options (SwiGLU clamp, probabilities before FC2).
inline bool mi355_numerics_options_enabled() { return true; }
// The 64-row tile configuration (two workgroups per CU) for grouped GEMMs whose groups average at
// most 32 rows (decode).
inline bool mi355_small_tiles_enabled() { return true; }
// Expert backward (bf16).
inline bool mi355_backward_enabled() { return true; }
// MegaGate RouteGrad (gradient of the routing weights with respect to the logits).
inline bool mi355_route_grad_enabled() { return true; }
// Dual-axis MX weight quantisation (col and row axes of the MXFP8 weight root in one pass).
inline bool mi355_mx_weight_prep_enabled() { return true; }
// MXFP8 expert backward (needs the MX K-contiguous GEMM path for its data-gradient GEMMs).
inline bool mi355_mx_backward_enabled() { return true; }
// The one-launch decode prologue (dispatch + MX token quantisation, decode_prep.h) of the MegaMoE
// forward on the 64-row tiles. Host-checked; until its GPU parity tests have passed it runs only
// while MI355MOE_DECODE_PREP=1 is set in the environment (read at each forward call, so a test can
// compare both prologues in one process).
inline bool mi355_decode_prep_enabled() {
  const char* v = getenv("MI355MOE_DECODE_PREP");
  return v != nullptr && strcmp(v, "1") == 0;
}
// The skinny 384 x 128 MX tile of the 8-wave GEMM for experts of 257..384 routed rows (one weight
// pass instead of two). Host-checked; until its GPU tests and an A/B have run it is used only while
// MI355MOE_PP_SKINNY=1 is set in the environment (read at each GEMM call).
inline bool mi355_pp_skinny_enabled() {
  const char* v = getenv("MI355MOE_PP_SKINNY");
  return v != nullptr && strcmp(v, "1") == 0;
}
