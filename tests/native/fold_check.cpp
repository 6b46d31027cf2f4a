// Host check of the append kernel's split absmax fold (test harness, built by
// tests/test_oracle.py). The kernel folds a 32-value block as four runs of 8
// values (FoldRun, csrc/tge_common.h) joined in order; the reference folds
// sequentially from +0 (quantize_kv_block, qwen2.cpp:88-93:
// `a = x >= 0 ? x : -x; if (!(maximum > a)) maximum = a`). Every block must
// give the same maximum bit for bit, NaN payloads and zero signs included.
//
//   fold_check <blocks> <seed>     prints one JSON line
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tge_common.h"

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float of_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static uint64_t state;
static uint32_t next_u32() {
  state ^= state << 13; state ^= state >> 7; state ^= state << 17;
  return (uint32_t)(state >> 11);
}

// One value drawn from a mix rich in the cases the fold must get right.
static float draw(float common) {
  const uint32_t k = next_u32() % 16;
  switch (k) {
    case 0: return 0.0f;
    case 1: return -0.0f;
    case 2: return of_bits(0x7FC00000u | (next_u32() & 0x803FFFFFu));  // NaN, either sign
    case 3: return of_bits(0x7F800001u | (next_u32() & 0x807FFFFFu));  // signalling-pattern NaN
    case 4: return (next_u32() & 1) ? __builtin_huge_valf() : -__builtin_huge_valf();
    case 5: return of_bits(next_u32() & 0x807FFFFFu);  // subnormal or zero
    case 6: case 7: return common;                     // ties
    case 8: return -common;
    default: return of_bits((next_u32() & 0x80000000u) | ((100u + next_u32() % 60u) << 23) | (next_u32() & 0x7FFFFFu));
  }
}

int main(int argc, char** argv) {
  const long blocks = argc > 1 ? atol(argv[1]) : 1000000;
  state = argc > 2 ? strtoull(argv[2], 0, 10) * 2654435761ull + 1 : 88172645463325252ull;
  long bad = 0, nan_blocks = 0, zero_blocks = 0;
  for (long n = 0; n < blocks; ++n) {
    float x[32];
    const float common = of_bits((100u + next_u32() % 60u) << 23 | (next_u32() & 0x7FFFFFu));
    const int mode = (int)(next_u32() % 4);
    for (int i = 0; i < 32; ++i) {
      if (mode == 0) x[i] = draw(common);                               // mixed specials
      else if (mode == 1) x[i] = (next_u32() & 1) ? 0.0f : -0.0f;          // zeros only
      else if (mode == 2) x[i] = (next_u32() % 8 == 0) ? draw(common) : common;
      else x[i] = of_bits(next_u32());                                   // any bit pattern
    }
    // reference order
    float m = 0.0f;
    bool any_nan = false;
    for (int i = 0; i < 32; ++i) {
      const float a = x[i] >= 0.0f ? x[i] : -x[i];
      if (!(m > a)) m = a;
      any_nan |= a != a;
    }
    // four runs of eight, joined in order
    tge::FoldRun all = tge::fold_run(x);
    for (int j = 1; j < 4; ++j) all = tge::fold_join(all, tge::fold_run(x + 8 * j));
    if (bits_of(all.v) != bits_of(m)) {
      if (bad < 5) fprintf(stderr, "block %ld: reference %08x, split %08x\n", n, bits_of(m), bits_of(all.v));
      ++bad;
    }
    nan_blocks += any_nan;
    zero_blocks += (m == 0.0f);
  }
  printf("{\"blocks\": %ld, \"mismatches\": %ld, \"blocks_with_nan\": %ld, \"zero_max_blocks\": %ld}\n",
         blocks, bad, nan_blocks, zero_blocks);
  return bad != 0;
}
