// fuzz_parsers.cpp — mutation fuzzing of the host-side parsers under
// AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU (test
// infrastructure; built and run by tests/test_sanitizers.py):
//
//   welvet_model_mount      the WMN1 model descriptor (model.cpp), including
//                           the store snapshots NWS1 exports carry
//   the wire tool's stdin   WVD1-3, WDB1, WVF1, WVN1, WVS1, WSB1, WSQ1, WRE1,
//                           SQB1, REB1 (wire_tool.cpp, its main() linked in
//                           as wire_tool_main)
//
// Both parse the whole message before any device work, so no GPU is needed:
// without one, a message that parses fails at its first device call.  From
// each seed (a valid message written by the test) the driver derives every
// prefix, every aligned 32-bit field replaced by boundary values, and random
// bit flips, byte insertions and deletions.  A run passes when no sanitizer
// fires (each report aborts), every mount returns a known status code with a
// terminated message, and every wire run exits 0, 1 or 2.
//
//   fuzz_parsers <report-prefix> <random-iterations> <rng-seed> <seed files...>
//   (*.wmn: descriptors, *.wire: wire tool input)
#include <sanitizer/common_interface_defs.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "welvet_c.h"

// wire_tool.cpp's main, compiled with -Dmain=wire_tool_main
int wire_tool_main(int argc, char **argv);

namespace {

using Bytes = std::vector<uint8_t>;

uint64_t g_rng = 1;
uint32_t rnd() {
  g_rng ^= g_rng >> 12;
  g_rng ^= g_rng << 25;
  g_rng ^= g_rng >> 27;
  return (uint32_t)((g_rng * 0x2545F4914F6CDD1Dull) >> 32);
}

const int32_t kBoundary[] = {0, 1, -1, 2, 3, 4, 7, 33, 4095, 4096, 4097, 65536, 1 << 26, (1 << 26) + 1,
                             0x7fffffff, (int32_t)0x80000000u, 0x40000000, 0x3f800000 /* 1.0f */,
                             0x7f800000 /* inf */, 0x7fc00000 /* nan */};

struct Tally {
  long runs = 0, codes[8] = {0};
};

bool read_file(const char *path, Bytes *out) {
  FILE *f = std::fopen(path, "rb");
  if (!f) return false;
  uint8_t buf[65536];
  size_t n;
  while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) out->insert(out->end(), buf, buf + n);
  std::fclose(f);
  return true;
}

bool ends_with(const std::string &s, const char *suffix) {
  const size_t n = std::strlen(suffix);
  return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

// welvet_model_mount on the bytes; false on an unexpected outcome
bool run_model(const Bytes &b, Tally *t) {
  welvet_model_session *s = nullptr;
  // a copy of exactly b.size() bytes, so a read past the end is reported
  uint8_t *copy = (uint8_t *)std::malloc(b.size() ? b.size() : 1);
  if (!b.empty()) std::memcpy(copy, b.data(), b.size());
  const welvet_status st = welvet_model_mount(copy, b.size(), &s);
  std::free(copy);
  if (s) welvet_model_release(s);
  ++t->runs;
  if (st.code < 0 || st.code > 7 || std::memchr(st.message, 0, sizeof st.message) == nullptr) {
    std::fprintf(stderr, "model: unexpected status %d\n", st.code);
    return false;
  }
  ++t->codes[st.code];
  return true;
}

// the wire tool's main on the bytes as stdin (stdout discarded)
bool run_wire(const Bytes &b, const std::string &tmp, Tally *t) {
  FILE *f = std::fopen(tmp.c_str(), "wb");
  if (!f) return false;
  if (!b.empty() && std::fwrite(b.data(), 1, b.size(), f) != b.size()) return false;
  std::fclose(f);
  if (!std::freopen(tmp.c_str(), "rb", stdin)) return false;
  char name[] = "welvet_dense_fwd";
  char *argv[] = {name, nullptr};
  const int rc = wire_tool_main(1, argv);
  std::fflush(stdout);
  ++t->runs;
  if (rc < 0 || rc > 2) {
    std::fprintf(stderr, "wire: unexpected exit code %d\n", rc);
    return false;
  }
  ++t->codes[rc];
  return true;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 5) {
    std::fprintf(stderr, "usage: fuzz_parsers <report-prefix> <iterations> <rng-seed> <seeds...>\n");
    return 2;
  }
  __sanitizer_set_report_path(argv[1]);
  const long iterations = std::atol(argv[2]);
  g_rng = std::strtoull(argv[3], nullptr, 10) | 1;
  const std::string tmp = std::string(argv[1]) + ".stdin";
  std::vector<std::pair<Bytes, bool>> seeds;  // (bytes, is model descriptor)
  for (int i = 4; i < argc; ++i) {
    Bytes b;
    if (!read_file(argv[i], &b)) {
      std::fprintf(stderr, "cannot read %s\n", argv[i]);
      return 2;
    }
    seeds.emplace_back(b, ends_with(argv[i], ".wmn"));
  }
  // the tool's replies and messages go nowhere; sanitizer reports go to files
  if (!std::freopen("/dev/null", "wb", stdout) || !std::freopen("/dev/null", "wb", stderr)) return 2;
  Tally model, wire;
  bool good = true;
  auto run = [&](const Bytes &b, bool is_model) {
    good = (is_model ? run_model(b, &model) : run_wire(b, tmp, &wire)) && good;
  };
  for (const auto &[seed, is_model] : seeds) {
    run(seed, is_model);
    // every prefix (the truncations a short read meets)
    for (size_t n = 0; n < seed.size(); ++n) run(Bytes(seed.begin(), seed.begin() + n), is_model);
    // every aligned 32-bit field set to each boundary value
    for (size_t at = 0; at + 4 <= seed.size(); at += 4)
      for (int32_t v : kBoundary) {
        Bytes b = seed;
        std::memcpy(b.data() + at, &v, 4);
        run(b, is_model);
      }
  }
  for (long it = 0; it < iterations && !seeds.empty(); ++it) {
    const auto &[seed, is_model] = seeds[rnd() % seeds.size()];
    Bytes b = seed;
    const int edits = 1 + (int)(rnd() % 4);
    for (int e = 0; e < edits; ++e) {
      switch (rnd() % 5) {
      case 0:  // bit flips
        if (!b.empty()) b[rnd() % b.size()] ^= (uint8_t)(1u << (rnd() % 8));
        break;
      case 1:  // an unaligned 32-bit field
        if (b.size() >= 4) {
          const int32_t v = kBoundary[rnd() % (sizeof kBoundary / sizeof kBoundary[0])];
          std::memcpy(b.data() + rnd() % (b.size() - 3), &v, 4);
        }
        break;
      case 2:  // insert bytes
        b.insert(b.begin() + (b.empty() ? 0 : rnd() % b.size()), 1 + rnd() % 16, (uint8_t)rnd());
        break;
      case 3:  // delete bytes
        if (!b.empty()) {
          const size_t at = rnd() % b.size(), n = std::min<size_t>(b.size() - at, 1 + rnd() % 16);
          b.erase(b.begin() + at, b.begin() + at + n);
        }
        break;
      default:  // truncate
        if (!b.empty()) b.resize(rnd() % b.size());
      }
    }
    run(b, is_model);
  }
  std::remove(tmp.c_str());
  FILE *out = std::fopen((std::string(argv[1]) + ".summary").c_str(), "w");
  if (out) {
    std::fprintf(out, "model runs %ld codes", model.runs);
    for (long c : model.codes) std::fprintf(out, " %ld", c);
    std::fprintf(out, "\nwire runs %ld exits %ld %ld %ld\n", wire.runs, wire.codes[0], wire.codes[1],
                 wire.codes[2]);
    std::fclose(out);
  }
  return good ? 0 : 1;
}
