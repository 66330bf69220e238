/*
 * TEST INFRASTRUCTURE ONLY - the CPU oracle for the MegaGate route. Only tests/, the smoke
 * check and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Plain-C restatement of the route semantics of MegaGate._torch_forward
 * (hyper_multicore/modules/mega_gate/module.py:189-227) and of the native route pipeline order
 * (hyper_multicore/ops/hyper_mega_gate/op_kernel/route_pipeline.h:104-130 compensated softplus,
 * :266-332 top-k, :334-538 gather / row-sum / +1e-20 / divide / scale), extended with the
 * DeepSeek-V3 group-limited selection, written to reproduce the gfx950 kernel's fp32 operation
 * order exactly:
 *   - exp / log are the deterministic Cody-Waite + polynomial forms (same constants, explicit
 *     fmaf, no contraction), so scores match bit for bit;
 *   - the softmax denominator is summed per lane (expert e -> lane e % 64, slot e / 64,
 *     ascending slots) and then combined by a 64-lane xor butterfly (masks 32,16,...,1);
 *   - selection: largest biased score, ties to the lower expert id; output in selection order;
 *   - renormalisation sums the selected unbiased scores in output order, adds 1e-20, divides,
 *     then multiplies by the scaling factor.
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -shared -fPIC router_ref.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LN2_HI 0.693145751953125f
#define LN2_LO 1.428606765330187e-06f

float oracle_det_expf(float x) {
  if (x != x) return x;
  if (x > 88.75f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, LN2_HI, x);
  r = fmaf(-n, LN2_LO, r);
  float p = 1.98412698e-04f;
  p = fmaf(p, r, 1.38888889e-03f);
  p = fmaf(p, r, 8.33333377e-03f);
  p = fmaf(p, r, 4.16666679e-02f);
  p = fmaf(p, r, 1.66666672e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

float oracle_det_logf(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? -INFINITY : NAN;
  if (isinf(x)) return x;
  uint32_t bits;
  memcpy(&bits, &x, 4);
  int e = (int)((bits >> 23) & 0xff) - 127;
  uint32_t mb = (bits & 0x7fffffu) | 0x3f800000u;
  float m;
  memcpy(&m, &mb, 4);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float z = s * s;
  float p = 0.15384615384615385f;
  p = fmaf(p, z, 0.18181818181818182f);
  p = fmaf(p, z, 0.22222222222222221f);
  p = fmaf(p, z, 0.2857142857142857f);
  p = fmaf(p, z, 0.4f);
  p = fmaf(p, z, 0.6666666666666666f);
  p = fmaf(p, z, 2.0f);
  float lm = s * p;
  float ef = (float)e;
  return fmaf(ef, LN2_HI, fmaf(ef, LN2_LO, lm));
}

static float score_one(float l, int scoring) {
  if (scoring == 1) return 1.0f / (1.0f + oracle_det_expf(-l));
  float e = oracle_det_expf(fminf(l, 20.0f));
  float u = e + 1.0f;
  float sp;
  if (u == 1.0f) {
    sp = e;
  } else {
    float ratio = e / (u - 1.0f);
    sp = oracle_det_logf(u) * ratio;
  }
  if (l > 20.0f) sp = l;
  return sqrtf(sp);
}

/* scoring: 0 softmax, 1 sigmoid, 2 sqrtsoftplus. Returns 0 on success. */
int oracle_route(const float* logits, int64_t T, int E, const float* bias, const float* bias_vl,
                 const uint8_t* mask, int K, int scoring, int G, int TG, float scale, float* weights,
                 int64_t* indices, float* scores_out) {
  if (E <= 0 || E > 1024 || K <= 0 || K > E || G < 1 || E % G) return -1;
  float* score = (float*)malloc(sizeof(float) * E);
  float* biased = (float*)malloc(sizeof(float) * E);
  unsigned char* taken = (unsigned char*)malloc(E);
  if (!score || !biased || !taken) return -2;
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    const float* b = (mask && bias_vl && mask[t]) ? bias_vl : bias;
    if (scoring == 0) {
      float mx = -INFINITY;
      for (int e = 0; e < E; ++e) mx = fmaxf(mx, l[e]);
      float part[64];
      for (int lane = 0; lane < 64; ++lane) {
        part[lane] = 0.0f;
        for (int e = lane; e < E; e += 64) {
          score[e] = oracle_det_expf(l[e] - mx);
          part[lane] = part[lane] + score[e];
        }
      }
      for (int m = 32; m >= 1; m >>= 1) {
        float nxt[64];
        for (int lane = 0; lane < 64; ++lane) nxt[lane] = part[lane] + part[lane ^ m];
        memcpy(part, nxt, sizeof(part));
      }
      for (int e = 0; e < E; ++e) score[e] = score[e] / part[0];
    } else {
      for (int e = 0; e < E; ++e) score[e] = score_one(l[e], scoring);
    }
    for (int e = 0; e < E; ++e) {
      biased[e] = score[e] + b[e];
      if (scores_out) scores_out[t * E + e] = score[e];
    }
    if (G > 1) {
      const int S = E / G;
      float gscore[64];
      unsigned char keep[64];
      for (int g = 0; g < G; ++g) {
        float t1 = -INFINITY, t2 = -INFINITY;
        for (int e = g * S; e < (g + 1) * S; ++e) {
          float v = biased[e];
          if (v > t1) { t2 = t1; t1 = v; } else if (v > t2) { t2 = v; }
        }
        gscore[g] = t1 + t2;
        keep[g] = 0;
      }
      for (int r = 0; r < TG; ++r) {
        int best = -1;
        for (int g = 0; g < G; ++g)
          if (!keep[g] && (best < 0 || gscore[g] > gscore[best])) best = g;
        keep[best] = 1;
      }
      for (int e = 0; e < E; ++e)
        if (!keep[e / S]) biased[e] = -INFINITY;
    }
    memset(taken, 0, E);
    float sum = 0.0f;
    float* w = weights + t * K;
    int64_t* idx = indices + t * K;
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (!taken[e] && (best < 0 || biased[e] > biased[best])) best = e;
      taken[best] = 1;
      idx[k] = best;
      w[k] = score[best];
    }
    if (K > 1) {
      for (int k = 0; k < K; ++k) sum = sum + w[k];
      float denom = sum + 1.0e-20f;
      for (int k = 0; k < K; ++k) w[k] = w[k] / denom;
    }
    for (int k = 0; k < K; ++k) w[k] = w[k] * scale;
  }
  free(score);
  free(biased);
  free(taken);
  return 0;
}

/*
 * Route backward with respect to the logits (RouteGrad), for the routing weights of oracle_route:
 *   s = score(l);  sel = s[idx];  D = sum_k sel + 1e-20 (K > 1);  w = (K > 1 ? sel / D : sel) * scale
 * in the operation order of torch autograd of that expression, which the reference's native
 * RouteGrad reproduces for sqrt-softplus (route_grad_pipeline.h:138-189: k0 = gw * scale, the
 * div backward cross term -k0 * ((sel / D) / D), a row sum, direct term k0 / D, their sum;
 * op_api/hyper_mega_gate_route_grad.cpp:109-120 and hyper_mega_gate_route_grad_post.cpp:68-141:
 * scatter-add into zeros, score * 2, RealDiv, SoftplusV2Grad with beta 1 and threshold 20):
 *   g_k   = K == 1 ? gw_k * scale : k0_k / D + sum_j (-k0_j * ((sel_j / D) / D))   (sum ascending j)
 *   sg_e  = 0 + g_k for e = idx_k, else 0
 *   sqrt-softplus: q = sg / (2 s);  out = l > 20 ? q : (q * z) / (z + 1),  z = exp(l)
 *   sigmoid:       out = (sg * (1 - s)) * s                     (torch sigmoid_backward)
 *   softmax:       out = s * (sg - sum_e sg_e s_e)              (torch softmax_backward_data; the sum
 *                                                                runs over the selected experts in
 *                                                                ascending k, the other terms are 0)
 * The softmax / sigmoid forms are torch autograd of MegaGate._torch_forward (module.py:199-227),
 * the reference's path for those scores. exp is oracle_det_expf (the kernel's). When accumulate
 * is nonzero the result is added to out (out = out + grad). Returns 0 on success.
 */
int oracle_route_grad(const float* logits, const float* scores, const int64_t* indices, const float* grad_w,
                      int64_t T, int E, int K, int scoring, float scale, int accumulate, float* out) {
  if (E <= 0 || K <= 0 || K > E || scoring < 0 || scoring > 2) return -1;
  float* sg = (float*)malloc(sizeof(float) * (size_t)E);
  float* g = (float*)malloc(sizeof(float) * (size_t)K);
  if (!sg || !g) return -2;
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    const float* s = scores + t * E;
    const int64_t* idx = indices + t * K;
    const float* gw = grad_w + t * K;
    if (K == 1) {
      g[0] = gw[0] * scale;
    } else {
      float sum = 0.0f;
      for (int k = 0; k < K; ++k) sum = sum + s[idx[k]];
      const float D = sum + 1.0e-20f;
      float row = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float k0 = gw[k] * scale;
        const float cross = (-k0) * ((s[idx[k]] / D) / D);
        row = row + cross;
      }
      for (int k = 0; k < K; ++k) g[k] = (gw[k] * scale) / D + row;
    }
    for (int e = 0; e < E; ++e) sg[e] = 0.0f;
    for (int k = 0; k < K; ++k) sg[idx[k]] = sg[idx[k]] + g[k];
    float dot = 0.0f;
    if (scoring == 0)
      for (int k = 0; k < K; ++k) dot = dot + g[k] * s[idx[k]];
    for (int e = 0; e < E; ++e) {
      float r;
      if (scoring == 2) {
        const float q = sg[e] / (2.0f * s[e]);
        if (l[e] > 20.0f) {
          r = q;
        } else {
          const float z = oracle_det_expf(l[e]);
          r = (q * z) / (z + 1.0f);
        }
      } else if (scoring == 1) {
        r = (sg[e] * (1.0f - s[e])) * s[e];
      } else {
        r = s[e] * (sg[e] - dot);
      }
      out[t * E + e] = accumulate ? out[t * E + e] + r : r;
    }
  }
  free(sg);
  free(g);
  return 0;
}
