// Host build of the direct-to-LDS GEMM's LDS layout maps (synaptik_amd/csrc/gemm_v2_layout.h), for
// both tile edges (BT = 128 and 64). Checks: the copy placement (chunk q <- source) and the
// fragment addressing (source -> LDS offset) are inverse bijections over a stage; the kernel's
// fragment offsets (a per-lane base plus compile-time block / k-row offsets, as gemm_v2.h forms
// them) equal the layout function; every 16-lane phase of a K-contiguous ds_read_b128 covers 16
// distinct 16-byte bank groups and every M/N-contiguous ds_read_b32 covers 64 distinct banks.
// Prints "ok" or the first failure.
#include <cstdio>
#include <vector>
#define __host__
#define __device__
#include "../synaptik_amd/csrc/gemm_v2_layout.h"

using namespace shk;

static int fail(const char* what, int bt, int a, int b, int c) {
  printf("FAIL %s BT=%d %d %d %d\n", what, bt, a, b, c);
  return 1;
}

static int check(int BT) {
  const int chunks = BT * 8, cpr = BT / 4, WT = BT / 2, NB = BT / 32;
  // 1. bijections
  std::vector<char> seen_k(BT * 8, 0), seen_m(32 * cpr, 0);
  for (int q = 0; q < chunks; ++q) {
    const int s = v2_kmaj_src(q), r = s >> 3, c = s & 7;
    if (r < 0 || r >= BT || seen_k[r * 8 + c]) return fail("kmaj src", BT, q, r, c);
    seen_k[r * 8 + c] = 1;
    if (v2_kmaj_off(r, c) != q * 4) return fail("kmaj off", BT, q, r, c);
    const int t = v2_mnmaj_src(q, cpr), k = t / cpr, cm = t % cpr;
    if (k < 0 || k >= 32 || seen_m[k * cpr + cm]) return fail("mnmaj src", BT, q, k, cm);
    seen_m[k * cpr + cm] = 1;
    for (int u = 0; u < 4; ++u)
      if (v2_mnmaj_off(k, 4 * cm + u, cpr) != q * 4 + u) return fail("mnmaj off", BT, q, k, u);
  }
  for (int w = 0; w < 2; ++w)
    for (int h = 0; h < 2; ++h)
      for (int B = 0; B < NB; ++B) {
        // 2. K-contiguous fragments: base[B & 1] + (B >> 1) * 1024
        for (int ph = 0; ph < 4; ++ph) {
          bool used[16] = {};
          for (int l = 16 * ph; l < 16 * ph + 16; ++l) {
            const int l16 = l & 15, g = l >> 4;
            const int off = v2_kmaj_off(w * WT + 16 * B + l16, 4 * h + g);
            const int base = v2_kmaj_off(w * WT + 16 * (B & 1) + l16, 4 * h + g) + (B >> 1) * 1024;
            if (off != base) return fail("kmaj frag", BT, w, h, B);
            const int grp = (off / 4) & 15;
            if (used[grp]) return fail("kmaj bank", BT, w, h, B);
            used[grp] = true;
          }
        }
        // 3. M/N-contiguous fragments: base (k = 4g) + (16 h + s) * BT
        for (int s = 0; s < 4; ++s) {
          bool used[64] = {};
          for (int l = 0; l < 64; ++l) {
            const int l16 = l & 15, g = l >> 4;
            const int off = v2_mnmaj_off(16 * h + 4 * g + s, w * WT + 16 * B + l16, cpr);
            const int base = v2_mnmaj_off(4 * g, w * WT + 16 * B + l16, cpr) + (16 * h + s) * BT;
            if (off != base) return fail("mnmaj frag", BT, w, h, B * 4 + s);
            if (used[off & 63]) return fail("mnmaj bank", BT, w, h, B * 4 + s);
            used[off & 63] = true;
          }
        }
      }
  return 0;
}

int main() {
  if (check(128) || check(64)) return 1;
  printf("ok\n");
  return 0;
}
