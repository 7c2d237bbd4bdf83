/* Exhaustive check of the division identity the quantize kernel uses for
 * scale = (wmax - wmin) / 15: for every float x in [2^-90, 2^126],
 *   y = x * fl(1/15);  q = fma(fma(-y, 15, x), fl(1/15), y)
 * equals the correctly rounded x / 15.  Exit status 0 when it holds. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
  const uint32_t lo = 0x12800000u, hi = 0x7E800000u; /* 2^-90 .. 2^126 */
  const float c = 1.0f / 15.0f;
  uint64_t bad = 0;
  for (uint32_t b = lo; b <= hi; ++b) {
    float x;
    memcpy(&x, &b, 4);
    volatile float ref = x / 15.0f;
    const float y = x * c;
    const float q = fmaf(fmaf(-y, 15.0f, x), c, y);
    if (q != ref) {
      if (bad < 10) printf("mismatch x=%a ref=%a q=%a\n", x, (double)ref, q);
      ++bad;
    }
  }
  printf("checked %u values, %llu mismatches\n", hi - lo + 1, (unsigned long long)bad);
  return bad != 0;
}
