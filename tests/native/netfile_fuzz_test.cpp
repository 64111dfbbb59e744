// The network-file reader (metalfish_amd/csrc/host/weights_file.cpp) on
// every committed fixture and on malformed variants of them -- TEST
// INFRASTRUCTURE ONLY.  Built with -fsanitize=address,undefined by
// tests/test_sanitizers.py, so an out-of-bounds read, a use after free,
// signed overflow or a misaligned load anywhere in the decoder aborts the run.
//
// Per fixture: LoadFile on the file itself; Parse on every prefix of its
// bytes (each copied into a heap buffer of exactly that size, so reading one
// byte past the end is caught); and Parse on seeded mutations (byte
// overwrites, bit flips, varint-length bumps, inserted and deleted bytes).
// Each call must either return or throw std::runtime_error / std::bad_alloc.
// Usage: netfile_fuzz_test FILE... ; prints a summary line and exits 0.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "weights_file.h"

namespace {

int g_ok = 0, g_rejected = 0, g_other = 0;

void TryParse(const std::vector<std::uint8_t> &bytes) {
  // An exactly sized heap copy: ASan flags any read past its end.
  std::unique_ptr<std::uint8_t[]> buf(new std::uint8_t[bytes.size() ? bytes.size() : 1]);
  if (!bytes.empty())
    std::memcpy(buf.get(), bytes.data(), bytes.size());
  try {
    mfh::wf::Weights w = mfh::wf::Parse(buf.get(), bytes.size());
    std::size_t n = 0;
    for (const auto &t : w.tensors)
      n += t.data.size();
    (void)n;
    ++g_ok;
  } catch (const std::runtime_error &) {
    ++g_rejected;
  } catch (const std::bad_alloc &) {
    ++g_rejected;
  } catch (const std::exception &e) {
    std::fprintf(stderr, "unexpected exception type: %s\n", e.what());
    ++g_other;
  }
}

bool ReadFile(const char *path, std::vector<std::uint8_t> &out) {
  std::FILE *f = std::fopen(path, "rb");
  if (!f)
    return false;
  std::uint8_t chunk[4096];
  std::size_t got;
  while ((got = std::fread(chunk, 1, sizeof(chunk), f)) > 0)
    out.insert(out.end(), chunk, chunk + got);
  std::fclose(f);
  return true;
}

}  // namespace

int main(int argc, char **argv) {
  std::uint32_t seed = 12345u;
  auto rnd = [&seed](std::uint32_t n) {
    seed = seed * 1664525u + 1013904223u;
    return n ? (seed >> 8) % n : 0u;
  };
  int files = 0;
  for (int a = 1; a < argc; ++a) {
    const std::string path = argv[a];
    try {
      mfh::wf::LoadFile(path);
      ++g_ok;
    } catch (const std::runtime_error &) {
      ++g_rejected;
    }
    std::vector<std::uint8_t> bytes;
    if (!ReadFile(argv[a], bytes)) {
      std::fprintf(stderr, "cannot read %s\n", argv[a]);
      return 2;
    }
    ++files;
    if (path.size() > 3 && path.compare(path.size() - 3, 3, ".gz") == 0)
      continue;  // compressed bytes: LoadFile above covers the gzip path
    for (std::size_t len = 0; len <= bytes.size(); ++len)
      TryParse(std::vector<std::uint8_t>(bytes.begin(), bytes.begin() + len));
    for (int m = 0; m < 2000 && !bytes.empty(); ++m) {
      std::vector<std::uint8_t> v = bytes;
      const int edits = 1 + static_cast<int>(rnd(3));
      for (int e = 0; e < edits; ++e) {
        const std::size_t at = rnd(static_cast<std::uint32_t>(v.size()));
        switch (rnd(5)) {
        case 0: v[at] = static_cast<std::uint8_t>(rnd(256)); break;
        case 1: v[at] ^= static_cast<std::uint8_t>(1u << rnd(8)); break;
        case 2: v[at] = static_cast<std::uint8_t>(v[at] | 0x80u); break;  // longer varint
        case 3: v.insert(v.begin() + at, static_cast<std::uint8_t>(rnd(256))); break;
        default:
          if (v.size() > 1)
            v.erase(v.begin() + at);
        }
      }
      TryParse(v);
    }
  }
  std::printf("netfile fuzz: %d files, %d parsed, %d rejected, %d unexpected\n", files, g_ok,
              g_rejected, g_other);
  return g_other == 0 && files > 0 ? 0 : 1;
}
