// Host-only driver for the .qw reader robustness test (tests/test_qw_fuzz.py): opens each file named on stdin,
// walks every tensor (name lookup, first and last byte of its data in the mapping) and the meta text, closes.
// Built with AddressSanitizer + UndefinedBehaviorSanitizer on the host side; no GPU call is made.
#include <cstdio>
#include <cstring>
#include <string>
#include <iostream>
#include "../include/kh.h"
int main() {
  std::string path;
  long ok = 0, bad = 0;
  char err[256];
  while (std::getline(std::cin, path)) {
    kh_qw* f = kh_qw_open(path.c_str(), err, sizeof err);
    if (!f) { bad++; continue; }
    ok++;
    const int n = kh_qw_count(f);
    volatile size_t sink = 0;
    for (int i = 0; i < n; i++) {
      kh_qw_tensor t;
      if (kh_qw_at(f, i, &t) == KH_OK) {
        sink += t.nbytes + t.ndim;
        if (t.host && t.nbytes) sink += ((const unsigned char*)t.host)[0] + ((const unsigned char*)t.host)[t.nbytes - 1];
        kh_qw_tensor u;
        kh_qw_find(f, t.name, &u);
      }
    }
    const char* m = kh_qw_meta(f);
    sink += m ? strlen(m) : 0;
    kh_qw_close(f);
  }
  printf("opened %ld rejected %ld\n", ok, bad);
  return 0;
}
