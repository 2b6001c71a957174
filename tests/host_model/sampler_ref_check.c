/* oracle/sampler_ref.c under AddressSanitizer / UndefinedBehaviorSanitizer
 * (built by tests/test_host_model.py with gcc): drives oracle_sample and
 * oracle_exp2_det over edge-case rows -- vocab sizes around the 512-element
 * segment and the 64-segment group boundaries, rows of -inf / NaN / +-huge
 * values, one finite entry, temperatures from 1e-30 to 1e30, uniforms 0 and
 * just below 1 -- and checks every drawn index lies in [0, V) and names an
 * entry that can be drawn (finite, or any index of a row with none).
 * Exit status 0 = all passed. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

float oracle_exp2_det(float t);
void oracle_sample(const float* logits, int64_t B, int64_t V, const float* temperature,
                   const float* uniform, int64_t* out);

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static float frand(void) {  /* uniform [0, 1) */
  rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17;
  return (float)((rng >> 40) & 0xffffff) / 16777216.0f;
}

int main(void) {
  int fails = 0;
  for (float t = -130.0f; t <= 0.0f; t += 0.37f) {
    const float e = oracle_exp2_det(t);
    if (!(e >= 0.0f && e <= 1.0f)) { fprintf(stderr, "exp2_det(%g) = %g\n", t, e); ++fails; }
  }
  if (oracle_exp2_det(NAN) != 0.0f || oracle_exp2_det(-INFINITY) != 0.0f) ++fails;
  const int64_t vocabs[] = {1, 2, 7, 511, 512, 513, 1023, 32767, 32768, 32769, 100000};
  const float temps[] = {1e-30f, 0.5f, 1.0f, 7.0f, 1e30f};
  const float unis[] = {0.0f, 0.25f, 0.999999f};
  for (size_t vi = 0; vi < sizeof(vocabs) / sizeof(vocabs[0]); ++vi) {
    const int64_t V = vocabs[vi];
    float* x = (float*)malloc(sizeof(float) * (size_t)V);
    for (int kind = 0; kind < 6; ++kind) {
      for (int64_t i = 0; i < V; ++i) {
        switch (kind) {
          case 0: x[i] = 8.0f * (frand() - 0.5f); break;                  /* ordinary */
          case 1: x[i] = -INFINITY; break;                                /* nothing drawable */
          case 2: x[i] = (i == V / 2) ? 3.0f : -INFINITY; break;         /* one finite entry */
          case 3: x[i] = (i % 3 == 0) ? NAN : frand(); break;             /* NaN holes */
          case 4: x[i] = (i % 2) ? 3.0e38f : -3.0e38f; break;             /* huge magnitudes */
          default: x[i] = (i % 5 == 0) ? -INFINITY : frand(); break;
        }
      }
      int any_finite = 0;
      for (int64_t i = 0; i < V; ++i) any_finite |= isfinite(x[i]) ? 1 : 0;
      for (size_t ti = 0; ti < 5; ++ti)
        for (size_t ui = 0; ui < 3; ++ui) {
          int64_t out = -7;
          oracle_sample(x, 1, V, &temps[ti], &unis[ui], &out);
          if (out < 0 || out >= V) {
            fprintf(stderr, "V=%lld kind=%d T=%g u=%g: index %lld\n", (long long)V, kind,
                    temps[ti], unis[ui], (long long)out);
            ++fails;
          } else if (any_finite && kind != 3 && !isfinite(x[out])) {
            fprintf(stderr, "V=%lld kind=%d: drew a non-finite entry\n", (long long)V, kind);
            ++fails;
          } else if (kind == 2 && out != V / 2) {
            fprintf(stderr, "V=%lld: one finite entry not drawn\n", (long long)V);
            ++fails;
          }
        }
    }
    free(x);
  }
  if (fails) { fprintf(stderr, "%d checks failed\n", fails); return 1; }
  printf("oracle sampler under sanitizers: all passed\n");
  return 0;
}
