// Evaluates covers() (diffrast_amd/csrc/coverage.h, the coverage test the visibility kernels
// run) on the CPU for a batch of (triangle, pixel centre) cases, so that its decisions can be
// compared with the oracle's. Input file: int32 n, then n records of 14 float32 (x0 x1 x2,
// y0 y1 y2, z0 z1 z2, w0 w1 w2, px, py). Output file: n records of (float32 covered, float32
// depth), depth 0 where not covered.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../diffrast_amd/csrc/coverage.h"

using namespace dr;

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  FILE* in = fopen(argv[1], "rb");
  FILE* out = fopen(argv[2], "wb");
  if (!in || !out) return 2;
  int32_t n = 0;
  if (fread(&n, sizeof n, 1, in) != 1) return 2;
  for (int32_t i = 0; i < n; ++i) {
    float r[14];
    if (fread(r, sizeof(float), 14, in) != 14) return 2;
    Tri T;
    for (int k = 0; k < 3; ++k) {
      T.x[k] = r[k];
      T.y[k] = r[3 + k];
      T.z[k] = r[6 + k];
      T.w[k] = r[9 + k];
    }
    T.reach_x = reach(T.x, T.w);
    T.reach_y = reach(T.y, T.w);
    float depth = 0.0f;
    const bool hit = covers(T.x, T.y, T.z, T.w, T.reach_x, T.reach_y, r[12], r[13], depth);
    const float rec[2] = {hit ? 1.0f : 0.0f, hit ? depth : 0.0f};
    fwrite(rec, sizeof(float), 2, out);
  }
  fclose(out);
  fclose(in);
  return 0;
}
