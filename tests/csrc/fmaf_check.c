/* Reads float32 triples (a, b, c) from stdin and writes fmaf(a, b, c), the
 * C library's correctly rounded fused multiply-add, for each.  The oracle's
 * float64 emulation (fma32) is checked against these results.            */
#include <math.h>
#include <stdio.h>

int main(void) {
  float t[3];
  while (fread(t, sizeof(float), 3, stdin) == 3) {
    const float r = fmaf(t[0], t[1], t[2]);
    fwrite(&r, sizeof(float), 1, stdout);
  }
  return 0;
}
