// Mutation fuzz of the C++ host API's snapshot readers (mlx-gen_amd/host/io.cpp), built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host code (tests/host_cpp/Makefile) and
// run on the CPU by tests/test_io_fuzz.py.  Test infrastructure, not part of the product.
//
// Seeds: a valid safetensors file (the golden fixture) and a config.json.  Each case mutates the
// header bytes (overwrite, insert a JSON token, erase, truncate; the 8-byte header length kept
// consistent with the edit half the time) and hands the file to read_safetensors, or mutates the
// config text and hands it to write_quantized_config.  Every outcome must be a parsed result or
// an mlxq::Error; a sanitizer report or any other exception aborts the run.
//
// usage: fuzz_io <fixture.safetensors> <scratch dir> <seed> <cases>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iterator>
#include <random>
#include <string>

#include "../../mlx-gen_amd/host/mlxq.hpp"

namespace {

const char* const kTokens[] = {"{", "}", "[", "]", ",", ":", "\"", "\\u00", "\\u", "\\", "1e999", "-1",
                               "18446744073709551616", "9223372036854775807", "-9223372036854775809",
                               "\"dtype\"", "\"U32\"", "\"BF16\"", "\"shape\"", "\"data_offsets\"",
                               "\"__metadata__\"", "null", "true", "false", "0", "1.5e-400", "[[[[[[[["};
constexpr int kNumTokens = sizeof(kTokens) / sizeof(kTokens[0]);

void write_file(const std::string& path, const std::string& bytes) {
  std::ofstream o(path, std::ios::binary);
  o.write(bytes.data(), (std::streamsize)bytes.size());
}

// Mutations inside [lo, hi) of s (hi > lo).
void mutate(std::string& s, size_t lo, size_t hi, std::mt19937_64& rng) {
  const int kind = (int)(rng() % 4);
  const int edits = 1 + (int)(rng() % 8);
  for (int m = 0; m < edits; ++m) {
    const size_t span = hi > lo ? hi - lo : 1;
    const size_t pos = std::min(s.size(), lo + (size_t)(rng() % span));
    if (kind == 0 && pos < s.size()) s[pos] = (char)(rng() & 0xff);
    else if (kind == 1) s.insert(pos, kTokens[rng() % kNumTokens]);
    else if (kind == 2 && pos < s.size()) s.erase(pos, 1 + (size_t)(rng() % 16));
    else if (kind == 3) {
      s.resize((size_t)(rng() % (s.size() + 1)));
      return;
    }
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 5) {
    fprintf(stderr, "usage: %s <fixture.safetensors> <scratch dir> <seed> <cases>\n", argv[0]);
    return 2;
  }
  std::ifstream f(argv[1], std::ios::binary);
  const std::string base((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (base.size() < 8) return 2;
  uint64_t n = 0;
  for (int k = 7; k >= 0; --k) n = (n << 8) | (uint8_t)base[k];
  const std::string dir = argv[2];
  const std::string st_path = dir + "/case.safetensors";
  const std::string cfg_dir = dir + "/cfg_src", out_dir = dir + "/cfg_out";
  std::filesystem::create_directories(cfg_dir);
  const std::string cfg_base =
      "{\"model_type\": \"qwen3\", \"hidden_size\": 3072, \"layers\": [1, 2.5, -3e2, true, null],\n"
      " \"name\": \"a\\u00e9\\n\\\"q\\\"\", \"nested\": {\"x\": [[], {}], \"y\": 1e-7}}";
  std::mt19937_64 rng(std::strtoull(argv[3], nullptr, 10));
  const long cases = std::strtol(argv[4], nullptr, 10);
  long parsed = 0, refused = 0;
  for (long it = 0; it < cases; ++it) {
    try {
      if (it % 4 != 3) {
        std::string s = base;
        mutate(s, 8, 8 + n, rng);
        if (s.size() >= 8 && (rng() & 1)) {  // header length consistent with the edit
          const uint64_t nn = n + s.size() - base.size();
          for (int k = 0; k < 8; ++k) s[k] = (char)((nn >> (8 * k)) & 0xff);
        }
        write_file(st_path, s);
        const mlxq::HostMap m = mlxq::read_safetensors(st_path);
        for (const auto& kv : m) {  // every tensor's bytes match its dtype and shape
          size_t count = 1;
          for (int64_t d : kv.second.shape) count *= (size_t)d;
          if (kv.second.data.size() != count * mlxq::dtype_size(kv.second.dtype)) {
            fprintf(stderr, "case %ld: %s holds %zu bytes for its shape\n", it, kv.first.c_str(),
                    kv.second.data.size());
            return 1;
          }
        }
      } else {
        std::string c = cfg_base;
        mutate(c, 0, c.size(), rng);
        write_file(cfg_dir + "/config.json", c);
        mlxq::write_quantized_config(cfg_dir, out_dir, 4, 64);
      }
      ++parsed;
    } catch (const mlxq::Error&) {
      ++refused;
    }
  }
  printf("fuzz_io seed %s: %ld cases, %ld parsed, %ld refused with mlxq::Error\n", argv[3], cases,
         parsed, refused);
  return 0;
}
