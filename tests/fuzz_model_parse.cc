// Mutation fuzzer for the engine's model front end (onnx.cc ParseModel,
// graph.cc BuildGraph and PropagateShapes) and the EP's partition (ep.cc
// EpPartition, EpRunBoundary, EpNodeKeys, EpRunModel and a build of each claimed
// run's model), built by tests/test_fuzz_cpu.py
// with AddressSanitizer and UndefinedBehaviorSanitizer on the host. Every
// mutated model must be accepted or refused with an error: a sanitizer report
// or a crash fails the run.
//
// usage: fuzz_model_parse SEED ITERATIONS MODEL.onnx...
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <iterator>
#include <string>
#include <unordered_map>
#include <vector>

#include "ep.h"
#include "graph.h"
#include "onnx.h"

namespace {

struct Rng {
  uint64_t s;
  uint32_t next() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return static_cast<uint32_t>(s >> 33);
  }
  uint32_t below(uint32_t n) { return n ? next() % n : 0; }
};

std::vector<unsigned char> mutate(const std::vector<unsigned char>& good, Rng& r) {
  std::vector<unsigned char> b = good;
  const int rounds = 1 + static_cast<int>(r.below(4));
  for (int k = 0; k < rounds && !b.empty(); ++k) {
    const size_t at = r.below(static_cast<uint32_t>(b.size()));
    switch (r.below(6)) {
      case 0:  // truncate
        b.resize(at);
        break;
      case 1:  // flip bits of a few bytes
        for (int i = 0, n = 1 + static_cast<int>(r.below(8)); i < n; ++i)
          b[r.below(static_cast<uint32_t>(b.size()))] ^= static_cast<unsigned char>(1u << r.below(8));
        break;
      case 2: {  // a special byte: continuation bit, zero, all ones
        static const unsigned char v[] = {0x00, 0x80, 0xff, 0x7f, 0x0a, 0x12};
        b[at] = v[r.below(6)];
        break;
      }
      case 3: {  // an oversized varint (a length or a count)
        static const unsigned char big[] = {0xff, 0xff, 0xff, 0xff, 0xff, 0xff, 0xff, 0xff, 0xff, 0x01};
        const size_t n = 1 + r.below(10);
        b.insert(b.begin() + static_cast<long>(at), big + 10 - n, big + 10);
        break;
      }
      case 4: {  // splice a slice of the model elsewhere
        const size_t from = r.below(static_cast<uint32_t>(b.size()));
        const size_t len = r.below(static_cast<uint32_t>(b.size() - from) + 1) % 512;
        std::vector<unsigned char> piece(b.begin() + static_cast<long>(from),
                                         b.begin() + static_cast<long>(from + len));
        b.insert(b.begin() + static_cast<long>(at), piece.begin(), piece.end());
        break;
      }
      default:  // delete a slice
        b.erase(b.begin() + static_cast<long>(at),
                b.begin() + static_cast<long>(at + r.below(static_cast<uint32_t>(b.size() - at) + 1) % 64));
        break;
    }
  }
  return b;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 4) {
    std::fprintf(stderr, "usage: %s SEED ITERATIONS MODEL...\n", argv[0]);
    return 2;
  }
  Rng rng{std::strtoull(argv[1], nullptr, 10)};
  const long iters = std::strtol(argv[2], nullptr, 10);
  long parsed = 0, built = 0, shaped = 0, claimed = 0, thrown = 0;
  for (int f = 3; f < argc; ++f) {
    std::ifstream in(argv[f], std::ios::binary);
    const std::vector<unsigned char> good((std::istreambuf_iterator<char>(in)), {});
    if (good.empty()) {
      std::fprintf(stderr, "cannot read %s\n", argv[f]);
      return 2;
    }
    for (long i = 0; i < iters; ++i) {
      const std::vector<unsigned char> b = mutate(good, rng);
      try {
        arthip::onnx::Model m;
        std::string err;
        if (!arthip::onnx::ParseModel(b.data(), b.size(), m, err)) continue;
        ++parsed;
        std::vector<arthip::EpRun> runs;
        if (arthip::EpPartition(m, runs, err)) {
          for (const arthip::EpRun& run : runs) {
            std::vector<std::string> acts, consts, outs, keys;
            arthip::onnx::Model sub;
            arthip::Graph sg;
            if (arthip::EpRunBoundary(m, run.nodes, acts, consts, outs, err) &&
                arthip::EpNodeKeys(m, run.nodes, keys, err) &&
                arthip::EpRunModel(m, run.nodes, sub, err) && arthip::BuildGraph(sub, sg, err))
              ++claimed;
          }
        }
        arthip::Graph g;
        if (!arthip::BuildGraph(m, g, err)) continue;
        ++built;
        std::unordered_map<std::string, arthip::Shape> shapes;
        const int64_t dims[][4] = {{1, 1, 16, 16}, {1, 3, 9, 7}, {2, 64, 5, 33}};
        for (const auto& d : dims) shaped += arthip::PropagateShapes(g, d, shapes) ? 1 : 0;
      } catch (const std::exception& e) {
        ++thrown;  // the C ABI turns these into error codes
      }
    }
  }
  std::printf("parsed %ld built %ld shaped %ld claimed %ld thrown %ld\n", parsed, built, shaped,
              claimed, thrown);
  return 0;
}
