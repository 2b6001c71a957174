/*
 * sampler_ref.c — CPU restatement of the fused sampler (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
 *
 * Greedy rows restate _argmax_kernel / torch.argmax (reference
 * litevllm/layers/sampler.py:60-84, 111-124): first index of the fp32 max.
 *
 * Temperature rows restate the build's inverse-CDF definition of
 * softmax(x / T) sampling at a supplied uniform u (the reference draws with
 * torch.multinomial, sampler.py:187, which no fixed vector can pin):
 *   c = log2(e) / T; 512-element segments; per segment max m_s, weights
 *   e_j = exp2_det((x_j - m_s) * c), 8-element lane chunks summed in order,
 *   Hillis-Steele inclusive scan over the 64 chunks; w_s = sigma_s *
 *   exp2_det((m_s - M) * c); groups of R = ceil(nseg/64) segments summed in
 *   order and scanned; target = u * S; four-level search (group, segment,
 *   chunk, element), each "first child whose cumulative value exceeds the
 *   target, else the last child with positive weight".
 * Compiled with -ffp-contract=off and without fast-math so every operation
 * is one IEEE fp32 operation in the written order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define SEG 512
#define LANES 64

/* exp2_det(t) for t <= 0 (every use): t < -200 and NaN are first replaced
 * by -200; n = floor(t), f = t - n (one IEEE subtraction; a result of 1.0,
 * which only t in (-2^-25, 0) can give, becomes the largest float below 1,
 * as the GPU's fract instruction clamps it); P(f) = 1 + f (c1 + f (c2 +
 * f (c3 + f (c4 + f c5)))) by fused multiply-adds, with c1..c5 a degree-5
 * minimax fit of 2^f on [0, 1) rounded to fp32; result ldexp(P(f), n), one
 * rounding (subnormal for n < -126, 0 below about -150).  Max relative error
 * over [-125, 0] < 2^-22.7 (every fp32 f in [0, 1) checked). */
float oracle_exp2_det(float t) {
  t = fmaxf(t, -200.0f); /* NaN -> -200 */
  const float n = floorf(t);
  float f = t - n;
  if (f >= 1.0f) f = 0x1.fffffep-1f;
  float q = 0x1.e974fap-10f;
  q = fmaf(q, f, 0x1.277856p-7f);
  q = fmaf(q, f, 0x1.c91ce6p-5f);
  q = fmaf(q, f, 0x1.ebdb5ap-3f);
  q = fmaf(q, f, 0x1.62e4bap-1f);
  const float p = fmaf(q, f, 1.0f);
  return ldexpf(p, (int)n);
}

/* In-place inclusive Hillis-Steele scan of 64 values: for d = 1, 2, ..., 32
 * every a[k] with k >= d becomes a[k] + a[k-d] (old values). */
static void hs_scan64(float* a) {
  float old[LANES];
  for (int d = 1; d < LANES; d <<= 1) {
    memcpy(old, a, sizeof old);
    for (int k = d; k < LANES; ++k) a[k] = old[k] + old[k - d];
  }
}

static float seg_elem(const float* x, int64_t V, int64_t i) {
  return i < V ? x[i] : -INFINITY;
}

/* Segment s: max, per-element weights e[512], chunk sums a[64], scan A[64]. */
static float segment_weights(const float* x, int64_t V, int s, float c, float* e, float* a,
                             float* A) {
  float ms = -INFINITY;
  for (int j = 0; j < SEG; ++j) ms = fmaxf(ms, seg_elem(x, V, (int64_t)s * SEG + j));
  for (int k = 0; k < LANES; ++k) {
    float acc = 0.0f;
    for (int j = 0; j < 8; ++j) {
      const float xv = seg_elem(x, V, (int64_t)s * SEG + 8 * k + j);
      const float ev = oracle_exp2_det((xv - ms) * c);
      e[8 * k + j] = ev;
      acc = acc + ev;
    }
    a[k] = acc;
  }
  memcpy(A, a, sizeof(float) * LANES);
  hs_scan64(A);
  return ms;
}

int64_t oracle_greedy_row(const float* x, int64_t V) {
  float bv = -INFINITY;
  int64_t bi = -1;
  for (int64_t i = 0; i < V; ++i)
    if (x[i] > bv) { bv = x[i]; bi = i; }
  return bi < 0 ? 0 : bi;
}

int64_t oracle_sample_row(const float* x, int64_t V, float temp, float u) {
  const float c = 0x1.715476p+0f / temp;
  if (!(temp > 0.0f) || !(c <= 3.0e38f)) return oracle_greedy_row(x, V);
  const int nseg = (int)((V + SEG - 1) / SEG);
  float* m = (float*)malloc(sizeof(float) * nseg);
  float* w = (float*)malloc(sizeof(float) * nseg);
  float e[SEG], a[LANES], A[LANES];
  for (int s = 0; s < nseg; ++s) {
    m[s] = segment_weights(x, V, s, c, e, a, A);
    w[s] = A[LANES - 1];
  }
  float M = -INFINITY;
  for (int s = 0; s < nseg; ++s) M = fmaxf(M, m[s]);
  const int R = (nseg + LANES - 1) / LANES;
  float b[LANES], B[LANES];
  for (int k = 0; k < LANES; ++k) {
    const int g0 = k * R < nseg ? k * R : nseg;
    const int g1 = g0 + R < nseg ? g0 + R : nseg;
    float acc = 0.0f;
    for (int s = g0; s < g1; ++s) {
      w[s] = w[s] * oracle_exp2_det((m[s] - M) * c);
      acc = acc + w[s];
    }
    b[k] = acc;
  }
  memcpy(B, b, sizeof B);
  hs_scan64(B);
  const float S = B[LANES - 1];
  int64_t result = 0;
  if (!(S > 0.0f)) goto done;
  {
    const float target = u * S;
    /* level 1 */
    int k = -1;
    for (int i = 0; i < LANES; ++i)
      if (B[i] > target && b[i] > 0.0f) { k = i; break; }
    if (k < 0)
      for (int i = 0; i < LANES; ++i)
        if (b[i] > 0.0f) k = i;
    const float base_k = (k == 0) ? 0.0f : B[k - 1];
    /* level 2 */
    const int t0 = k * R < nseg ? k * R : nseg;
    const int t1 = t0 + R < nseg ? t0 + R : nseg;
    int sstar = -1;
    float base = 0.0f, acc = base_k;
    for (int s = t0; s < t1; ++s) {
      const float nxt = acc + w[s];
      if (nxt > target) { sstar = s; base = acc; break; }
      acc = nxt;
    }
    if (sstar < 0) {
      acc = base_k;
      for (int s = t0; s < t1; ++s) {
        if (w[s] > 0.0f) { sstar = s; base = acc; }
        acc = acc + w[s];
      }
    }
    /* level 3 */
    segment_weights(x, V, sstar, c, e, a, A);
    const float scale = oracle_exp2_det((m[sstar] - M) * c);
    int kk = -1;
    for (int i = 0; i < LANES; ++i)
      if ((base + A[i] * scale > target) && a[i] > 0.0f) { kk = i; break; }
    if (kk < 0)
      for (int i = 0; i < LANES; ++i)
        if (a[i] > 0.0f) kk = i;
    /* level 4 */
    float q = (kk == 0) ? 0.0f : A[kk - 1];
    int jstar = -1;
    for (int j = 0; j < 8; ++j) {
      q = q + e[8 * kk + j];
      if (jstar < 0 && e[8 * kk + j] > 0.0f && base + q * scale > target) jstar = j;
    }
    if (jstar < 0)
      for (int j = 0; j < 8; ++j)
        if (e[8 * kk + j] > 0.0f) jstar = j;
    result = (int64_t)sstar * SEG + kk * 8 + jstar;
  }
done:
  free(m);
  free(w);
  return result;
}

/* Row-batched entry: logits fp32 [B, V] (row stride V). */
void oracle_sample(const float* logits, int64_t B, int64_t V, const float* temperature,
                   const float* uniform, int64_t* out) {
  for (int64_t r = 0; r < B; ++r)
    out[r] = oracle_sample_row(logits + r * V, V, temperature[r], uniform ? uniform[r] : 0.0f);
}
