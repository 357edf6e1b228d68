/*
 * router_ref.c — CPU oracle (test infrastructure only, never on the product
 * path) for the routing and dispatch stages of FusionLLM's DeepSeekMoE.
 *
 * oracle_router_fwd restates DeepSeekMoE._route, models/moe.py:44-50:
 *   logits = gate(x)                          moe.py:46
 *   scores = sigmoid(logits)                  moe.py:47
 *   weights, indices = topk(scores, k)        moe.py:48
 *   weights = weights / (sum + 1e-10) * rs    moe.py:49
 * with the router precision of the build: the logits are accumulated in fp32
 * from bf16 operands (the reference module, in bf16, rounds logits and scores
 * to bf16), exact ties go to the lowest expert index, NaN ranks above every
 * number.  The fp32 summation order is the one the gfx950 kernel uses
 * (16 lane partials over 8-element chunks, then an xor butterfly), and the
 * exponential is the same Cody-Waite + degree-7 Taylor evaluation, so the
 * kernel's indices, weights and scores are reproduced bit for bit.
 *
 * oracle_dispatch restates the permutation of
 * DeepSeekMoE._dispatch_scatter_gather, models/moe.py:55-64: a stable sort of
 * the flattened expert indices (torch.argsort; the reference's sort is
 * stable at T*k >= 32768), per-expert counts and the exclusive scan.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float pow2i(int n) { /* 2^n for -126 <= n <= 127 */
  uint32_t u = (uint32_t)(n + 127) << 23;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* e^x: x = n*ln2 + r with |r| <= ln2/2 (Cody-Waite split of ln2), e^r by its
 * degree-7 Taylor polynomial in Horner form, scaling by 2^n in two halves. */
float oracle_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541016f) return 0.0f;
  const float n = rintf(x * 1.4426950216293335f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.4286067653302598e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2;
  const int n2 = ni - n1;
  return (p * pow2i(n1)) * pow2i(n2);
}

float oracle_sigmoid(float l) { return 1.0f / (1.0f + oracle_expf(-l)); }

static int beats(float a, float b) {
  const int an = a != a, bn = b != b;
  if (an || bn) return an && !bn;
  return a > b;
}

/* fp32 logit of token row xr against gate row wr, in the kernel's order. */
static float logit_fp32(const uint16_t* xr, const uint16_t* wr, int64_t dim) {
  float p[16];
  const int64_t nchunk = dim / 8;
  for (int j = 0; j < 16; ++j) {
    float acc = 0.0f;
    for (int64_t c = j; c < nchunk; c += 16)
      for (int i = 0; i < 8; ++i) acc = fmaf(bf2f(xr[c * 8 + i]), bf2f(wr[c * 8 + i]), acc);
    p[j] = acc;
  }
  for (int off = 8; off >= 1; off >>= 1) {
    float q[16];
    for (int j = 0; j < 16; ++j) q[j] = p[j] + p[j ^ off];
    memcpy(p, q, sizeof p);
  }
  return p[0];
}

/* x [T,dim], gate_w [E,dim], gate_b [E] as bf16 bit patterns.  Outputs
 * idx/weights/topv [T,k]; logits/scores [T,E] when non-NULL. */
int oracle_router_fwd(const uint16_t* x, const uint16_t* gate_w, const uint16_t* gate_b, int64_t T,
                      int64_t dim, int E, int k, float route_scale, int32_t* idx, float* weights,
                      float* topv, float* logits, float* scores) {
  if (dim % 8 != 0 || E < 1 || E > 64 || k < 1 || k > E || k > 8) return 1;
  for (int64_t t = 0; t < T; ++t) {
    float s[64];
    for (int e = 0; e < E; ++e) {
      const float l = logit_fp32(x + t * dim, gate_w + (int64_t)e * dim, dim) + bf2f(gate_b[e]);
      s[e] = oracle_sigmoid(l);
      if (logits) logits[t * E + e] = l;
      if (scores) scores[t * E + e] = s[e];
    }
    uint64_t taken = 0;
    float val[8];
    int sel[8];
    for (int j = 0; j < k; ++j) {
      int best = -1;
      float bv = 0.0f;
      for (int e = 0; e < E; ++e) {
        if ((taken >> e) & 1ull) continue;
        if (best < 0 || beats(s[e], bv)) { best = e; bv = s[e]; }
      }
      taken |= 1ull << best;
      sel[j] = best;
      val[j] = bv;
    }
    float sum = val[0];
    for (int j = 1; j < k; ++j) sum = sum + val[j];
    const float denom = sum + 1e-10f;
    for (int j = 0; j < k; ++j) {
      idx[t * k + j] = sel[j];
      weights[t * k + j] = (val[j] / denom) * route_scale;
      topv[t * k + j] = val[j];
    }
  }
  return 0;
}

/* Counting sort of the T*k slots by expert, stable in slot order.
 * counts [E], offsets [E+1], perm [T*k] (row -> slot), pos [T*k] (slot -> row). */
int oracle_dispatch(const int32_t* idx, int64_t T, int E, int k, int32_t* counts, int32_t* offsets,
                    int32_t* perm, int32_t* pos) {
  const int64_t n = T * k;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int64_t s = 0; s < n; ++s) {
    if (idx[s] < 0 || idx[s] >= E) return 1;
    counts[idx[s]]++;
  }
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  int32_t fill[64];
  for (int e = 0; e < E; ++e) fill[e] = offsets[e];
  for (int64_t s = 0; s < n; ++s) {
    const int32_t r = fill[idx[s]]++;
    perm[r] = (int32_t)s;
    pos[s] = r;
  }
  return 0;
}
