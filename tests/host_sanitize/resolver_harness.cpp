// Host harness for the mapping resolver (furiosa-opt_amd/csrc/mapping.cpp), built with AddressSanitizer
// and UndefinedBehaviorSanitizer by tests/test_host_sanitizers.py. It drives every entry point that
// takes caller input -- the MappingSerde JSON parser, the m![..] text parser, the offset parser --
// and the resolution steps behind fo_transpose / fo_reduce / fo_contraction (flatten, sequence,
// carve, window_base, strides), on valid mappings and on a deterministic stream of malformed JSON
// (truncations, byte flips, insertions, deep nesting, oversized numbers). A malformed input must end
// in a thrown exception, never in a sanitizer report. Prints "ok <cases>" on success.
#include <cstdint>
#include <cstdio>
#include <exception>
#include <map>
#include <string>
#include <vector>

#include "mapping.hpp"

using namespace fo::mapping;

namespace {

uint64_t rng_state = 0x9e3779b97f4a7c15ull;
uint64_t next_rand() {  // splitmix64
  uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

long cases = 0, rejected = 0;

// Every resolution step on one parsed mapping and a partner of the same axes.
void exercise(const NodeP& m, const NodeP& other) {
  Factors f = flatten(m), g = flatten(other);
  (void)size(f);
  (void)strides(f);
  (void)is_padding(f);
  (void)to_json(unflatten(f));
  try { (void)remove_padding(f); } catch (const std::exception&) {}
  try { (void)first_axis(f); } catch (const std::exception&) {}
  try { (void)broadcast_symbols(f, g); } catch (const std::exception&) {}
  for (Mode mode : {Mode::Read, Mode::Write, Mode::Carve}) {
    try {
      Joint j = sequence({f}, {g}, mode);
      for (const Wheel& w : j.wheels) (void)w.stride.at(0);
    } catch (const std::exception&) {}
  }
  try { (void)carve(f, g); } catch (const std::exception&) {}
  std::map<std::string, int64_t> origin;
  for (const std::string& s : idents(m)) origin[s] = 0;
  try { (void)window_base(f, origin); } catch (const std::exception&) {}
}

void parse_and_exercise(const std::string& json, const NodeP& partner) {
  ++cases;
  try {
    NodeP m = parse_json(json);
    exercise(m, partner ? partner : m);
    NodeP back = parse_json(to_json(m));  // round trip
    if (to_json(back) != to_json(m)) {
      std::fprintf(stderr, "round trip changed %s\n", json.c_str());
      std::exit(2);
    }
  } catch (const std::exception&) {
    ++rejected;
  }
}

}  // namespace

int main() {
  const std::map<std::string, int64_t> sizes = {{"A", 6}, {"B", 4}, {"C", 64}, {"I", 512}, {"J", 512},
                                               {"K", 64}, {"N", 8}, {"G", 2}, {"D", 128}, {"T", 512}};
  const std::vector<std::pair<std::string, std::string>> texts = {
      {"A, B", "B, A"},
      {"A # 8, B", "B, A"},
      {"B # 8, A # 7", "A, B"},
      {"C / 8, C % 8", "C"},
      {"1, 1 # 2, I / 32, J / 32, I % 32, K", "I, K"},
      {"1, 1 # 2, I / 32, J / 32, J % 8, J / 8 % 4, K / 16, K % 16", "J, K"},
      {"N, G, T / 16, D, T % 16", "N, G, T, D"},
      {"T, N, D", "N, G, T"},
      {"N, G, D", "N, G"},
      {"C = 32, B", "C, B"},
  };
  std::vector<std::string> seeds;
  for (const auto& [a, b] : texts) {
    NodeP ma = parse_text(a, sizes), mb = parse_text(b, sizes);
    ++cases;
    exercise(ma, mb);
    exercise(mb, ma);
    seeds.push_back(to_json(ma));
    seeds.push_back(to_json(mb));
    parse_and_exercise(seeds.back(), ma);
  }
  // malformed text mappings and offsets
  for (const char* bad : {"", "A,", "A / 0", "A % 0", "A # -3", "Q", "A, A", "(A", "A / 7", "A # 99999999999999999999"}) {
    ++cases;
    try { (void)parse_text(bad, sizes); } catch (const std::exception&) { ++rejected; }
  }
  for (const char* off : {"{}", "{\"A\": 3}", "{\"A\": -1}", "{\"A\": 1e400}", "{\"A\": \"x\"}", "{\"A\": 3", "[1, 2]",
                          "{\"A\": 9223372036854775808}", "{\"\\ud800\": 1}", "{\"A\": 1, \"A\": 2}"}) {
    ++cases;
    try { (void)parse_offset_json(off); } catch (const std::exception&) { ++rejected; }
  }
  // deep nesting at and beyond the parser's depth limit
  for (int depth : {10, 255, 256, 257, 5000}) {
    std::string s;
    for (int i = 0; i < depth; ++i) s += "{\"Stride\": {\"inner\": ";
    s += "{\"Symbol\": {\"symbol\": \"A\", \"size\": 6}}";
    for (int i = 0; i < depth; ++i) s += ", \"stride\": 1}}";
    parse_and_exercise(s, nullptr);
  }
  // byte-level mutations of the valid seeds
  const std::string alphabet = "{}[]\":,0123456789-+.eE\\u\"abcdefSymbolStridePairleft";
  for (int round = 0; round < 100000; ++round) {
    std::string s = seeds[next_rand() % seeds.size()];
    const int edits = 1 + (int)(next_rand() % 4);
    for (int e = 0; e < edits && !s.empty(); ++e) {
      const size_t pos = next_rand() % s.size();
      switch (next_rand() % 5) {
        case 0: s.erase(pos, 1 + next_rand() % 4); break;                        // delete
        case 1: s.insert(pos, 1, alphabet[next_rand() % alphabet.size()]); break;  // insert
        case 2: s[pos] = alphabet[next_rand() % alphabet.size()]; break;          // replace
        case 3: s.resize(pos); break;                                             // truncate
        default: s.insert(pos, "99999999999999999999"); break;                    // oversized number
      }
    }
    parse_and_exercise(s, nullptr);
  }
  std::printf("ok %ld cases, %ld rejected\n", cases, rejected);
  return 0;
}
