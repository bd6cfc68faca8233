/* Exhaustive check of the division-free code rule of the bf16 quantiser
 * (quant_snap8 in compact_amd/csrc/glu_math.h):
 *
 *   rint(fma(v, rs, 3072) - 3072) == rint(fp32(v / safe))
 *
 * for every bf16 v with 2^-8 <= |v / safe| < 256, every positive finite fp16
 * safe (subnormals included), and rs = fp32(1 / safe) moved by 0, +-1 and
 * +-2 ulp (the GPU's v_rcp_f32 is within 1 ulp).  Quotients below 2^-8 give
 * code 0 under both (|y - 3072| < 2^-8 + 2^-14).  The second rounding is done
 * as the kernel does it: adding 1.5 * 2^23 - 3072 and reading the integer.
 *
 * Test infrastructure: built and run by tests/test_quant_snap_rule.py.
 * Prints "ok <cases>" and exits 0, or prints the first failures and exits 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#ifndef CPT_SNAP_GRID
#define CPT_SNAP_GRID 3072.0f
#endif

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float f16_to_f32(uint16_t h) {
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  if (e == 0) return ldexpf((float)m, -24);
  return ldexpf((float)(m | 0x400), (int)e - 25);
}

int main(void) {
  /* the fused multiply-add must round once */
  volatile float a = 1.0f + 0x1p-23f;
  if (fmaf(a, a, -1.0f) != 0x1p-22f + 0x1p-46f) {
    printf("fmaf is not fused\n");
    return 2;
  }
  const float kGrid = CPT_SNAP_GRID, kInt = 12582912.0f;
  long long cases = 0, bad = 0;
  for (uint32_t h = 1; h < 0x7C00; ++h) {           /* positive finite fp16 */
    const float s = f16_to_f32((uint16_t)h);
    float rs[5];
    rs[2] = 1.0f / s;
    rs[1] = nextafterf(rs[2], 0.0f);
    rs[0] = nextafterf(rs[1], 0.0f);
    rs[3] = nextafterf(rs[2], INFINITY);
    rs[4] = nextafterf(rs[3], INFINITY);
    /* bf16 patterns (upper halves of fp32) with 2^-8 s <= v < 256 s */
    const uint32_t lo = u_of(ldexpf(s, -8)) >> 16, hi = (u_of(256.0f * s) >> 16) + 1;
    for (uint32_t b = lo; b <= hi; ++b) {
      for (int sign = 0; sign < 2; ++sign) {
        const float v = f_of((b << 16) | (sign ? 0x80000000u : 0u));
        const float q = v / s;
        if (!(fabsf(q) < 256.0f) || fabsf(q) < 0x1p-8f) continue;
        const float want = rintf(q);
        for (int k = 0; k < 5; ++k) {
          const float y = fmaf(v, rs[k], kGrid);
          volatile float z = y + (kInt - kGrid);
          const float got = z - kInt;
          ++cases;
          if (got != want) {
            if (bad < 10)
              printf("v %.9g safe %.9g rs %+d ulp: got %g want %g\n", v, s, k - 2, got, want);
            ++bad;
          }
        }
      }
    }
  }
  if (bad) {
    printf("FAIL %lld of %lld\n", bad, cases);
    return 1;
  }
  printf("ok %lld\n", cases);
  return 0;
}
