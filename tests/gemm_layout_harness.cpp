// Host build of the large-problem GEMM's LDS layout maps (synaptik_amd/csrc/gemm_v2_layout.h).
// Checks: the copy placement (chunk q <- source) and the fragment addressing (source -> LDS
// offset) are inverse bijections over a stage; the kernel's precomputed fragment offsets (lane
// base + compile-time block / k-row offsets, as written in gemm_v2.h) equal the layout function;
// every 16-lane phase of a K-contiguous ds_read_b128 covers 16 distinct 16-byte bank groups and
// every M/N-contiguous ds_read_b32 covers 64 distinct banks. Prints "ok" or the first failure.
#include <cstdio>
#define __host__
#define __device__
#include "../synaptik_amd/csrc/gemm_v2_layout.h"

using namespace shk;

static int fail(const char* what, int a, int b, int c) {
  printf("FAIL %s %d %d %d\n", what, a, b, c);
  return 1;
}

int main() {
  // 1. bijections
  static bool seen_k[128][8], seen_m[32][32];
  for (int q = 0; q < 1024; ++q) {
    const int s = v2_kmaj_src(q), r = s >> 3, c = s & 7;
    if (r < 0 || r >= 128 || seen_k[r][c]) return fail("kmaj src", q, r, c);
    seen_k[r][c] = true;
    if (v2_kmaj_off(r, c) != q * 4) return fail("kmaj off", q, r, c);
    const int t = v2_mnmaj_src(q), k = t >> 5, cm = t & 31;
    if (k < 0 || k >= 32 || seen_m[k][cm]) return fail("mnmaj src", q, k, cm);
    seen_m[k][cm] = true;
    for (int u = 0; u < 4; ++u)
      if (v2_mnmaj_off(k, 4 * cm + u) != q * 4 + u) return fail("mnmaj off", q, k, u);
  }
  for (int w = 0; w < 2; ++w)
    for (int h = 0; h < 2; ++h)
      for (int B = 0; B < 4; ++B) {
        // 2. K-contiguous fragments: base[B & 1] + (B >> 1) * 1024
        for (int ph = 0; ph < 4; ++ph) {
          bool used[16] = {};
          for (int l = 16 * ph; l < 16 * ph + 16; ++l) {
            const int l16 = l & 15, g = l >> 4;
            const int off = v2_kmaj_off(w * 64 + 16 * B + l16, 4 * h + g);
            const int base = v2_kmaj_off(w * 64 + 16 * (B & 1) + l16, 4 * h + g) + (B >> 1) * 1024;
            if (off != base) return fail("kmaj frag", w, h, B);
            const int grp = (off / 4) & 15;
            if (used[grp]) return fail("kmaj bank", w, h, B);
            used[grp] = true;
          }
        }
        // 3. M/N-contiguous fragments: 512 g + 64 w + 16 (B ^ g) + l16 + (16 h + s) * 128
        for (int s = 0; s < 4; ++s) {
          bool used[64] = {};
          for (int l = 0; l < 64; ++l) {
            const int l16 = l & 15, g = l >> 4;
            const int off = v2_mnmaj_off(16 * h + 4 * g + s, w * 64 + 16 * B + l16);
            const int base = 512 * g + 64 * w + 16 * (B ^ g) + l16 + (16 * h + s) * 128;
            if (off != base) return fail("mnmaj frag", w, h, B * 4 + s);
            if (used[off & 63]) return fail("mnmaj bank", w, h, B * 4 + s);
            used[off & 63] = true;
          }
        }
      }
  printf("ok\n");
  return 0;
}
