// Host-only driver for the GGUF reader of libseeker_hip (seeker_amd/csrc/
// gguf.cpp), built with AddressSanitizer + UBSan by tests/test_gguf.py.
//
//   gguf_fuzz FILE...            inspect each file, print "<status> <message>"
//   gguf_fuzz --mutate N SEED F  inspect N deterministic mutations of F
//                                (byte overwrites, 64-bit field stores,
//                                truncations), print a status histogram
//
// Each parse reads a heap copy of exactly the file's bytes, so any read past
// the end is an ASan report. Exit status 0 unless a sanitizer aborts.
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/seeker_hip.h"

static char g_err[1024];
void sh_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

static std::vector<uint8_t> slurp(const char* path) {
  std::vector<uint8_t> b;
  FILE* f = std::fopen(path, "rb");
  if (!f) return b;
  uint8_t buf[1 << 16];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + n);
  std::fclose(f);
  return b;
}

static int inspect(const std::vector<uint8_t>& img) {
  // exact-size heap copy: one byte past the end is outside the allocation
  uint8_t* p = (uint8_t*)std::malloc(img.empty() ? 1 : img.size());
  if (!img.empty()) std::memcpy(p, img.data(), img.size());
  sh_model_dims d;
  g_err[0] = 0;
  const int rc = sh_gguf_inspect(p, img.size(), &d);
  std::free(p);
  return rc;
}

static uint64_t splitmix(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int main(int argc, char** argv) {
  if (argc >= 5 && std::strcmp(argv[1], "--mutate") == 0) {
    const long n = std::atol(argv[2]);
    uint64_t s = std::strtoull(argv[3], nullptr, 10);
    const std::vector<uint8_t> base = slurp(argv[4]);
    if (base.size() < 64) return 2;
    // mutations land in the header and tensor table, where the parser reads
    const size_t hdr = base.size() < 4096 ? base.size() : 4096;
    long hist[8] = {0};
    for (long i = 0; i < n; ++i) {
      std::vector<uint8_t> m = base;
      const int kind = (int)(splitmix(&s) % 4);
      const size_t at = (size_t)(splitmix(&s) % hdr);
      if (kind == 0) {
        m[at] = (uint8_t)splitmix(&s);
      } else if (kind == 1 && at + 8 <= m.size()) {
        static const uint64_t vals[] = {0, 1, 0xFFFFFFFFull, 0xFFFFFFFFFFFFFFFFull, 0x8000000000000000ull,
                                        1ull << 32, 1ull << 40, 0x7FFFFFFFFFFFFFFFull};
        const uint64_t v = vals[splitmix(&s) % 8];
        std::memcpy(&m[at], &v, 8);
      } else if (kind == 2) {
        m.resize(at);
      } else {
        for (int j = 0; j < 4; ++j) m[(size_t)(splitmix(&s) % hdr)] ^= (uint8_t)(1u << (splitmix(&s) % 8));
      }
      const int rc = inspect(m);
      hist[rc >= 0 && rc < 8 ? rc : 7]++;
    }
    for (int i = 0; i < 8; ++i) std::printf("%d %ld\n", i, hist[i]);
    return 0;
  }
  for (int i = 1; i < argc; ++i) {
    const int rc = inspect(slurp(argv[i]));
    std::printf("%d %s\n", rc, g_err);
  }
  return 0;
}
