/*
 * Exhaustive check of a float->half converter over all 2^32 float bit
 * patterns (test harness, built by tests/test_oracle.py).
 *
 *   f16_sweep <candidate.so> <symbol> [<reference.so> <symbol>]
 *
 * For every input x it compares the candidate with the hardware F16C
 * conversion in round-to-nearest-even mode, which is an independent model:
 * the reference recipe (kernels.hpp:358-386) must differ from RNE exactly on
 *   - ties (dropped bits == 100...0) whose truncated result is even: RNE
 *     keeps it, the recipe rounds the magnitude up (result = RNE + 1);
 *   - 2^-25 < |x| < 2^-24: the recipe flushes to signed zero, RNE gives the
 *     smallest subnormal;
 *   - NaN: the recipe returns sign|0x7E00 whatever the payload.
 * Any other difference, or a difference of the wrong form, is counted as a
 * violation. With a second library it also counts inputs where the two
 * converters differ at all. Prints one JSON line.
 */
#include <dlfcn.h>
#include <immintrin.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

typedef uint16_t (*conv_fn)(float);

static int predicted(uint32_t u, uint16_t rne, uint16_t* expect) {
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t biased = (u >> 23) & 0xFFu;
  const uint32_t frac = u & 0x7FFFFFu;
  if (biased == 0xFFu && frac) { *expect = (uint16_t)(sign | 0x7E00u); return 1; }
  if (biased == 0xFFu) return 0;
  const int e = (int)biased - 127;
  if (e == -25 && frac != 0) { *expect = (uint16_t)sign; return 1; }
  if (e < -24 || e > 15) return 0;
  uint32_t sig, drop;
  if (e < -14) { sig = 0x800000u | frac; drop = (uint32_t)(-14 - e) + 13u; }
  else { sig = frac; drop = 13u; }
  const uint32_t rest = sig & ((1u << drop) - 1u);
  const uint32_t kept = e < -14 ? (sig >> drop) : (frac >> 13);
  if (rest == (1u << (drop - 1u)) && (kept & 1u) == 0u) {
    *expect = (uint16_t)(rne + 1u);
    return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc != 3 && argc != 5) return 2;
  void* h1 = dlopen(argv[1], RTLD_NOW);
  if (!h1) { fprintf(stderr, "%s\n", dlerror()); return 2; }
  conv_fn cand = (conv_fn)dlsym(h1, argv[2]);
  conv_fn other = NULL;
  if (argc == 5) {
    void* h2 = dlopen(argv[3], RTLD_NOW);
    if (!h2) { fprintf(stderr, "%s\n", dlerror()); return 2; }
    other = (conv_fn)dlsym(h2, argv[4]);
  }
  if (!cand || (argc == 5 && !other)) return 2;
  unsigned long long violations = 0, ties = 0, tiny = 0, nans = 0, same = 0, vs_other = 0;
  long long first_bad = -1;
#pragma omp parallel for reduction(+:violations,ties,tiny,nans,same,vs_other) schedule(static, 1 << 20)
  for (long long i = 0; i < (1LL << 32); ++i) {
    const uint32_t u = (uint32_t)i;
    float x;
    memcpy(&x, &u, 4);
    const uint16_t c = cand(x);
    const uint16_t rne = (uint16_t)_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT);
    uint16_t expect = rne;
    const int differs = predicted(u, rne, &expect);
    if (c != expect) {
      ++violations;
      if (first_bad < 0) first_bad = i;
    } else if (differs) {
      const uint32_t biased = (u >> 23) & 0xFFu;
      if (biased == 0xFFu) ++nans;
      else if ((int)biased - 127 == -25) ++tiny;
      else ++ties;
    } else {
      ++same;
    }
    if (other && other(x) != c) ++vs_other;
  }
  printf("{\"violations\": %llu, \"ties_up\": %llu, \"tiny_flush\": %llu, \"nan\": %llu, "
         "\"same_as_rne\": %llu, \"vs_other\": %lld, \"first_bad\": %lld}\n",
         violations, ties, tiny, nans, same, other ? (long long)vs_other : -1LL, first_bad);
  return 0;
}
