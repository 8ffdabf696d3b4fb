/* Host-only robustness check of the oracle's safetensors reader (oracle/oracle.c), built with
 * ASan and UBSan by tests/test_parser_sanitizers.py. Opens ITERS mutated copies of the header
 * of the checkpoint in DIR (truncations, garbled bytes, bogus header lengths, structural
 * characters), then checks that the restored original still loads. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/oracle.h"

static uint64_t s = 88172645463325252ull;
static uint64_t rnd(void) {
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  return s;
}

static int load(const char* path) {
  int st = 0;
  char err[256];
  or_model* m = or_load_model(path, &st, err, sizeof err);
  if (!m) return 0;
  or_free_model(m);
  return 1;
}

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  char path[1024];
  snprintf(path, sizeof path, "%s/model.safetensors", argv[1]);
  const int iters = atoi(argv[2]);
  FILE* f = fopen(path, "rb");
  if (!f) return 2;
  fseek(f, 0, SEEK_END);
  const long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* orig = malloc((size_t)n);
  if (fread(orig, 1, (size_t)n, f) != (size_t)n) return 2;
  fclose(f);
  if (!load(path)) return 3;
  uint64_t hl;
  memcpy(&hl, orig, 8);
  int ok = 0;
  for (int it = 0; it < iters; it++) {
    char* buf = malloc((size_t)n);
    memcpy(buf, orig, (size_t)n);
    long len = n;
    switch (it % 5) {
      case 0: len = (long)(rnd() % (8 + hl + 64)); break;
      case 1: for (int k = 0; k < 8; k++) buf[8 + rnd() % hl] = (char)rnd(); break;
      case 2: { uint64_t v = rnd(); memcpy(buf, &v, 8); break; }
      case 3: { uint64_t v = hl + rnd() % 64 - 32; memcpy(buf, &v, 8); break; }
      default: buf[8 + rnd() % hl] = "{}[]\":,"[rnd() % 7]; break;
    }
    FILE* o = fopen(path, "wb");
    fwrite(buf, 1, (size_t)len, o);
    fclose(o);
    free(buf);
    ok += load(path);
  }
  FILE* o = fopen(path, "wb");
  fwrite(orig, 1, (size_t)n, o);
  fclose(o);
  free(orig);
  if (!load(path)) return 3;
  printf("accepted %d of %d mutated files\n", ok, iters);
  return 0;
}
