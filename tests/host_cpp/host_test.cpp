// host_test.cpp — tests of the C++ host API (mlx-gen_amd/host/mlxq.hpp), run by pytest.
//
//   host_test cpu   file formats and host logic only (no device work)
//   host_test gpu   the API end to end on the GPU, checked against the reference's golden fixture
//                   (tests/golden/quant_q4q8.safetensors, read through the API's own reader) and
//                   the CPU oracle (oracle/liboracle.so; test infrastructure, linked here only)
//
// Mirrors the reference's tests/quant_parity.rs (packing bit-exact, dequantize bit-exact,
// quantized_matmul within tolerance) and adds the layer and loader seams of src/adapters.rs,
// src/nn.rs and src/quant.rs.  Prints one line per case and exits non-zero on the first failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include <unistd.h>

#include "../../include/mlxq.h"
#include "../../mlx-gen_amd/host/mlxq.hpp"

extern "C" {
float oracle_bf16_round(float x);
int oracle_quantize(const float* w, int64_t N, int64_t K, int gs, int bits, int sb_bf16, uint32_t* wq,
                    float* scales, float* biases);
int oracle_dequantize(const uint32_t* wq, const float* scales, const float* biases, int64_t N, int64_t K,
                      int gs, int bits, int out_bf16, float* out);
int oracle_qmm(const float* x, int64_t M, int64_t K, const uint32_t* wq, const float* scales,
               const float* biases, int64_t N, int gs, int bits, int w_bf16, int out_bf16, float* y);
float oracle_silu(float v, int out_bf16);
float oracle_fp16_round(float x);
int oracle_linear(const float* x, int64_t M, int64_t K, const uint32_t* wq, const float* scales,
                  const float* biases, int64_t N, int gs, int bits, int w_bf16, int x_bf16,
                  int sb_bf16, const float* bias, int bias_bf16, const float* lora_a,
                  const float* lora_b, int64_t rank, int lora_bf16, float lora_scale, int act,
                  float* y, int* out_bf16);
int oracle_lokr_residual(const float* x, int64_t M, int64_t K, const float* delta, int64_t N,
                         float scale, int x_bf16, const float* y_in, int y_bf16, float* y,
                         int* out_bf16);
}

namespace fs = std::filesystem;
using namespace mlxq;

static int g_failures = 0;
#define EXPECT(cond, ...)                                            \
  do {                                                               \
    if (!(cond)) {                                                   \
      fprintf(stderr, "FAIL %s:%d: %s: ", __FILE__, __LINE__, #cond); \
      fprintf(stderr, __VA_ARGS__);                                  \
      fprintf(stderr, "\n");                                         \
      ++g_failures;                                                  \
    }                                                                \
  } while (0)

static void banner(const char* name) {
  printf("[case] %s\n", name);
  fflush(stdout);
}

// ---- host-side helpers ---------------------------------------------------------------------------
static std::vector<float> bf16_normal(std::mt19937& rng, size_t n, float std_) {
  std::normal_distribution<float> d(0.0f, std_);
  std::vector<float> v(n);
  for (auto& x : v) x = oracle_bf16_round(d(rng));
  return v;
}
static std::vector<uint16_t> to_bf16_bits(const std::vector<float>& v) {
  std::vector<uint16_t> o(v.size());
  for (size_t i = 0; i < v.size(); ++i) {
    uint32_t u;
    memcpy(&u, &v[i], 4);
    o[i] = (uint16_t)(u >> 16);  // values are already bf16-exact
  }
  return o;
}
static std::vector<float> from_bf16_bits(const uint16_t* p, size_t n) {
  std::vector<float> o(n);
  for (size_t i = 0; i < n; ++i) {
    uint32_t u = (uint32_t)p[i] << 16;
    memcpy(&o[i], &u, 4);
  }
  return o;
}
template <typename T>
static std::vector<T> host(const Array& a) {
  std::vector<T> v(a.nbytes() / sizeof(T));
  a.to_host(v.data());
  return v;
}
static std::vector<float> host_f32(const Array& a) {
  if (a.dtype() == Dtype::Bfloat16) {
    auto b = host<uint16_t>(a);
    return from_bf16_bits(b.data(), b.size());
  }
  return host<float>(a);
}
// IEEE binary16 bits of a value that fp16 represents exactly (oracle_fp16_round's outputs).
static uint16_t fp16_bits_exact(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const float a = std::fabs(f);
  if (a == 0.0f) return sign;
  int e;
  std::frexp(a, &e);  // a = m 2^e, m in [0.5, 1)
  if (e - 1 < -14) return (uint16_t)(sign | (uint16_t)std::ldexp(a, 24));  // subnormal: a / 2^-24
  const uint32_t mant = (uint32_t)std::ldexp(a, 11 - e) - 1024u;           // 10 fraction bits
  return (uint16_t)(sign | (uint16_t)(((e - 1 + 15) << 10) | mant));
}
static Array bf16_array(const std::vector<float>& v, std::vector<int64_t> shape) {
  auto b = to_bf16_bits(v);
  return Array::from_host(b.data(), shape, Dtype::Bfloat16);
}
static double rel_fro(const std::vector<float>& y, const std::vector<float>& r) {
  double num = 0, den = 0;
  for (size_t i = 0; i < y.size(); ++i) {
    num += ((double)y[i] - r[i]) * ((double)y[i] - r[i]);
    den += (double)r[i] * r[i];
  }
  return std::sqrt(num / std::max(den, 1e-300));
}
static fs::path repo_root(const char* argv0) {
  return fs::absolute(fs::path(argv0)).parent_path().parent_path().parent_path();
}

// ---- CPU cases -------------------------------------------------------------------------------------
static void cpu_cases(const fs::path& root) {
  const fs::path tmp = fs::temp_directory_path() / ("mlxq_host_test_" + std::to_string(::getpid()));
  fs::create_directories(tmp);

  banner("stacked expert packs: detection, bits, axis-0 split (host only)");
  {
    Weights w;
    char* base = reinterpret_cast<char*>(0x100000);  // never dereferenced: shape logic only
    w["m.experts.gate_up_proj.weight"] = Array::borrow(base, {3, 8, 16}, Dtype::Uint32);  // K=128 Q4
    w["m.experts.gate_up_proj.scales"] = Array::borrow(base, {3, 8, 2}, Dtype::Bfloat16);
    w["m.experts.gate_up_proj.biases"] = Array::borrow(base, {3, 8, 2}, Dtype::Bfloat16);
    w["m.experts.gate_up_proj_bias"] = Array::borrow(base, {3, 8}, Dtype::Bfloat16);
    EXPECT(has_packed_experts(w, "m", "gate_up") && !has_packed_experts(w, "m", "down"), "detection");
    StackedExperts st = load_packed_experts(w, "m", "gate_up");
    EXPECT(st.bits == 4 && st.group_size == 64 && st.num_experts() == 3, "bits/group/E");
    std::vector<QuantizedLinear> parts = st.split();
    EXPECT(parts.size() == 3 && parts[2].weight.shape() == std::vector<int64_t>({8, 16}) &&
               parts[2].in_features() == 128, "split shapes");
    EXPECT((char*)parts[2].weight.data() - base == 2 * 8 * 16 * 4 &&
               (char*)parts[1].bias->data() - base == 8 * 2, "split offsets");
    bool threw = false;
    try { load_packed_experts(w, "m", "down"); } catch (const Error&) { threw = true; }
    EXPECT(threw, "missing stack throws");
  }

  banner("safetensors round trip, every dtype");
  {
    HostMap m;
    const Dtype dts[] = {Dtype::Float32, Dtype::Bfloat16, Dtype::Uint32, Dtype::Int32, Dtype::Float16,
                         Dtype::Int64, Dtype::Uint8, Dtype::Int8, Dtype::Float64, Dtype::Bool};
    int k = 0;
    for (Dtype dt : dts) {
      HostTensor t;
      t.dtype = dt;
      t.shape = {3, 5};
      t.data.resize(15 * dtype_size(dt));
      for (size_t i = 0; i < t.data.size(); ++i) t.data[i] = (uint8_t)(i * 7 + k);
      m["t." + std::string(dtype_name(dt))] = t;
      ++k;
    }
    HostTensor empty;
    empty.dtype = Dtype::Float32;
    empty.shape = {0, 4};
    m["empty"] = empty;
    write_safetensors((tmp / "a.safetensors").string(), m);
    HostMap back = read_safetensors((tmp / "a.safetensors").string());
    EXPECT(back.size() == m.size(), "%zu tensors back", back.size());
    for (const auto& [name, t] : m) {
      EXPECT(back.count(name) == 1, "%s missing", name.c_str());
      EXPECT(back[name].dtype == t.dtype && back[name].shape == t.shape && back[name].data == t.data,
             "%s differs", name.c_str());
    }
    // the data section starts 8-byte aligned
    std::ifstream f(tmp / "a.safetensors", std::ios::binary);
    uint64_t n = 0;
    f.read((char*)&n, 8);
    EXPECT(n % 8 == 0, "header length %llu", (unsigned long long)n);
  }

  banner("golden fixture through read_safetensors");
  {
    HostMap g = read_safetensors((root / "tests" / "golden" / "quant_q4q8.safetensors").string());
    EXPECT(g.at("w").dtype == Dtype::Float32 && g.at("w").shape == std::vector<int64_t>({128, 256}), "w");
    EXPECT(g.at("q4.wq").dtype == Dtype::Uint32 && g.at("q4.wq").shape == std::vector<int64_t>({128, 32}), "q4.wq");
    EXPECT(g.at("q8.wq").shape == std::vector<int64_t>({128, 64}), "q8.wq");
    EXPECT(g.at("q4.scales").shape == std::vector<int64_t>({128, 4}), "q4.scales");
    // codes recomputed on the CPU from the fixture's own w match its packed words
    std::vector<uint32_t> wq(128 * 32);
    std::vector<float> s(128 * 4), b(128 * 4);
    EXPECT(oracle_quantize((const float*)g.at("w").data.data(), 128, 256, 64, 4, 0, wq.data(), s.data(),
                           b.data()) == 0, "oracle_quantize");
    EXPECT(memcmp(wq.data(), g.at("q4.wq").data.data(), wq.size() * 4) == 0, "q4 words");
  }

  banner("malformed files are errors");
  {
    std::ofstream(tmp / "short.safetensors", std::ios::binary) << "abc";
    bool threw = false;
    try { read_safetensors((tmp / "short.safetensors").string()); } catch (const Error&) { threw = true; }
    EXPECT(threw, "short file accepted");
    std::string bad = std::string("\x10\0\0\0\0\0\0\0", 8) + "{\"x\":{\"dtype\":\"Q9\"}}";
    bad.resize(8 + 16);
    std::ofstream(tmp / "bad.safetensors", std::ios::binary) << bad;
    threw = false;
    try { read_safetensors((tmp / "bad.safetensors").string()); } catch (const Error&) { threw = true; }
    EXPECT(threw, "malformed header accepted");
    threw = false;
    try { dtype_from_name("C64"); } catch (const Error&) { threw = true; }
    EXPECT(threw, "unknown dtype accepted");
    // Headers that are well-formed bytes but wrong JSON shapes or values: every one is an
    // mlxq::Error with MLXQ_EINVAL, never another exception type or a crash.
    const std::vector<std::string> headers = {
        "{\"x\":{\"dtype\":\"F32\",\"shape\":4,\"data_offsets\":[0,16]}}",          // shape not a list
        "{\"x\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":\"0\"}}",       // offsets not a list
        "{\"x\":{\"dtype\":\"F32\",\"shape\":[-4],\"data_offsets\":[0,16]}}",       // negative dim
        "{\"x\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":[0,99999999999999999999]}}",
        "{\"x\":{\"dtype\":\"F32\",\"shape\":[4294967296,4294967296],\"data_offsets\":[0,16]}}",
        "{\"x\":{\"dtype\":\"F\\uZZ32\",\"shape\":[4],\"data_offsets\":[0,16]}}",   // bad \\u escape
        "{\"x\":{\"dtype\":\"F32\",\"shape\":[4],\"data_offsets\":[0,1.5e999]}}",
        std::string(5000, '[') + std::string(5000, ']'),                          // deep nesting
    };
    for (size_t h = 0; h < headers.size(); ++h) {
      std::string file(8, '\0');
      const uint64_t n = headers[h].size();
      for (int k = 0; k < 8; ++k) file[k] = (char)(n >> (8 * k));
      file += headers[h] + std::string(16, '\0');
      std::ofstream(tmp / "bad2.safetensors", std::ios::binary) << file;
      int status = -1;
      try {
        read_safetensors((tmp / "bad2.safetensors").string());
      } catch (const Error& e) {
        status = e.status;
      } catch (...) {
        status = -2;
      }
      EXPECT(status == MLXQ_EINVAL, "malformed header %zu gave status %d", h, status);
    }
  }

  banner("write_quantized_config merges into an existing config");
  {
    fs::create_directories(tmp / "src");
    std::ofstream(tmp / "src" / "config.json")
        << "{\"hidden_size\": 3072, \"name\": \"a\\\"b\", \"ratio\": 0.5, \"layers\": [1, 2],"
           " \"nested\": {\"ok\": true, \"none\": null}, \"quantization\": {\"bits\": 8}}";
    write_quantized_config((tmp / "src").string(), (tmp / "dst").string(), 4, 64);
    std::ifstream f(tmp / "dst" / "config.json");
    std::string text((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    EXPECT(text.find("\"hidden_size\": 3072") != std::string::npos, "%s", text.c_str());
    EXPECT(text.find("\"name\": \"a\\\"b\"") != std::string::npos, "%s", text.c_str());
    EXPECT(text.find("\"layers\": [1,2]") != std::string::npos, "%s", text.c_str());
    EXPECT(text.find("\"bits\": 4") != std::string::npos && text.find("\"group_size\": 64") != std::string::npos &&
               text.find("\"bits\": 8") == std::string::npos, "%s", text.c_str());
    write_quantized_config((tmp / "nothing").string(), (tmp / "dst2").string(), 8, 32);
    std::ifstream f2(tmp / "dst2" / "config.json");
    std::string t2((std::istreambuf_iterator<char>(f2)), std::istreambuf_iterator<char>());
    EXPECT(t2.find("\"quantization\"") != std::string::npos && t2.find("\"group_size\": 32") != std::string::npos,
           "%s", t2.c_str());
  }
  fs::remove_all(tmp);
}

// ---- GPU cases -------------------------------------------------------------------------------------
static void gpu_cases(const fs::path& root) {
  const HostMap g = read_safetensors((root / "tests" / "golden" / "quant_q4q8.safetensors").string());
  const auto& hw = g.at("w");
  const auto& hx = g.at("x");

  for (int bits : {4, 8}) {
    banner(bits == 4 ? "golden quantize/dequantize/qmm Q4" : "golden quantize/dequantize/qmm Q8");
    const std::string p = "q" + std::to_string(bits) + ".";
    Array w = Array::from_host(hw.data.data(), hw.shape, hw.dtype);
    Packed q = quantize(w, 64, bits);
    EXPECT(q.wq.dtype() == Dtype::Uint32 && q.wq.shape() == g.at(p + "wq").shape, "wq shape");
    EXPECT(host<uint8_t>(q.wq) == g.at(p + "wq").data, "packed words differ from the fixture");
    EXPECT(host<uint8_t>(q.scales) == g.at(p + "scales").data, "scales differ from the fixture");
    EXPECT(host<uint8_t>(q.biases) == g.at(p + "biases").data, "biases differ from the fixture");
    Array deq = dequantize(q.wq, q.scales, q.biases, 64, bits);
    EXPECT(host<uint8_t>(deq) == g.at(p + "deq").data, "dequantize differs from the fixture");
    Array x = Array::from_host(hx.data.data(), hx.shape, hx.dtype);
    Array y = quantized_matmul(x, q.wq, q.scales, q.biases, true, 64, bits);
    const auto ref = g.at(p + "qmm");
    std::vector<float> r(ref.data.size() / 4);
    memcpy(r.data(), ref.data.data(), ref.data.size());
    const double e = rel_fro(host<float>(y), r);
    EXPECT(e < 1e-5, "relFro %.3e", e);
    EXPECT(packed_bits(q.wq, q.scales, 64) == bits, "packed_bits");
    bool threw = false;
    try { quantized_matmul(x, q.wq, q.scales, q.biases, false, 64, bits); } catch (const Error& err) {
      threw = err.status == 2;  // MLXQ_EUNSUPPORTED
    }
    EXPECT(threw, "transpose=false accepted");
  }

  banner("AdaptableLinear on an fp16 stream (SDXL): bf16-cast base and bias, f32 result");
  {
    // mlx-gen-sdxl/src/model.rs:216,283-296: fp16 activations through AdaptableLinear::quantize's
    // bf16 packs; MLX promotes fp16 against bf16 to f32, so the product, bias add and result are f32.
    std::mt19937 rng(11);
    const int64_t M = 77, K = 768, N = 320;
    std::vector<float> wf(N * K), bias(N), x(M * K);
    std::normal_distribution<float> nw(0.0f, 0.02f), nx(0.0f, 1.0f);
    for (auto& v : wf) v = nw(rng);
    for (auto& v : bias) v = nw(rng) * 10.0f;
    for (auto& v : x) v = oracle_fp16_round(nx(rng));
    std::vector<uint16_t> xh(x.size());
    for (size_t i = 0; i < x.size(); ++i) xh[i] = fp16_bits_exact(x[i]);
    AdaptableLinear l = AdaptableLinear::dense(Array::from_host(wf.data(), {N, K}, Dtype::Float32),
                                               Array::from_host(bias.data(), {N}, Dtype::Float32));
    l.quantize(4, std::nullopt);
    EXPECT(l.out_dtype(Dtype::Float16) == Dtype::Float32, "fp16 x promotes to f32");
    Array y = l.forward(Array::from_host(xh.data(), {M, K}, Dtype::Float16));
    EXPECT(y.dtype() == Dtype::Float32 && y.shape() == std::vector<int64_t>({M, N}), "fp16 forward output");
    std::vector<float> wb(wf.size()), bias_b(N), ref(M * N);
    for (size_t i = 0; i < wf.size(); ++i) wb[i] = oracle_bf16_round(wf[i]);
    for (int64_t n = 0; n < N; ++n) bias_b[n] = oracle_bf16_round(bias[n]);
    std::vector<uint32_t> wq(N * K / 8);
    std::vector<float> sc(N * K / 64), zb(N * K / 64);
    oracle_quantize(wb.data(), N, K, 64, 4, 1, wq.data(), sc.data(), zb.data());
    int out_bf16 = -1;
    oracle_linear(x.data(), M, K, wq.data(), sc.data(), zb.data(), N, 64, 4, 0, 0, 1, bias_b.data(), 1,
                  nullptr, nullptr, 0, 1, 1.0f, 0, ref.data(), &out_bf16);
    EXPECT(out_bf16 == 0, "oracle result dtype");
    const double e = rel_fro(host<float>(y), ref);
    EXPECT(e < 2e-5, "relFro %.3e", e);
  }

  banner("AdaptableLinear: bf16 cast + quantize, bias, two LoRA adapters");
  {
    std::mt19937 rng(7);
    const int64_t M = 37, K = 256, N = 192, R1 = 16, R2 = 24;
    std::vector<float> wf(N * K);
    std::normal_distribution<float> nd(0.0f, 0.02f);
    for (auto& v : wf) v = nd(rng);  // f32 weights: quantize() casts to bf16 first
    std::vector<float> bias = bf16_normal(rng, N, 0.1f), x = bf16_normal(rng, M * K, 1.0f);
    std::vector<float> a1 = bf16_normal(rng, K * R1, 0.01f), b1 = bf16_normal(rng, R1 * N, 0.01f);
    std::vector<float> a2 = bf16_normal(rng, K * R2, 0.01f), b2 = bf16_normal(rng, R2 * N, 0.01f);
    AdaptableLinear l = AdaptableLinear::dense(Array::from_host(wf.data(), {N, K}, Dtype::Float32),
                                               Array::from_host(bias.data(), {N}, Dtype::Float32));
    bool threw = false;
    try { l.forward(bf16_array(x, {M, K})); } catch (const Error&) { threw = true; }
    EXPECT(threw, "dense forward should be refused");
    l.quantize(4, std::nullopt);
    EXPECT(l.is_quantized() && l.quantized().group_size == 64 && l.base_shape()[1] == K, "quantize");
    l.push(Adapter{bf16_array(a1, {K, R1}), bf16_array(b1, {R1, N}), 0.75f});
    l.push(Adapter{bf16_array(a2, {K, R2}), bf16_array(b2, {R2, N}), 1.5f});
    Array y = l.forward(bf16_array(x, {M, K}).reshape({1, M, K}));
    EXPECT(y.shape() == std::vector<int64_t>({1, M, N}) && y.dtype() == Dtype::Bfloat16, "output shape");
    // reference: bf16-cast weights, quantize, linear with bias + adapter 1, then + adapter 2
    std::vector<float> wb(wf.size());
    for (size_t i = 0; i < wf.size(); ++i) wb[i] = oracle_bf16_round(wf[i]);
    std::vector<uint32_t> wq(N * K / 8);
    std::vector<float> s(N * K / 64), z(N * K / 64), ref(M * N);
    oracle_quantize(wb.data(), N, K, 64, 4, 1, wq.data(), s.data(), z.data());
    EXPECT(host<uint32_t>(l.quantized().weight) == wq, "packed words");
    std::vector<float> bias_b(N);
    for (int64_t n = 0; n < N; ++n) bias_b[n] = oracle_bf16_round(bias[n]);
    oracle_linear(x.data(), M, K, wq.data(), s.data(), z.data(), N, 64, 4, M > 8, 1, 1, bias_b.data(), 1,
                  a1.data(), b1.data(), R1, 1, 0.75f, 0, ref.data(), nullptr);
    std::vector<float> xa(M * R2);
    for (int64_t m = 0; m < M; ++m)
      for (int64_t r = 0; r < R2; ++r) {
        double acc = 0;
        for (int64_t k = 0; k < K; ++k) acc += (double)x[m * K + k] * a2[k * R2 + r];
        xa[m * R2 + r] = oracle_bf16_round((float)acc);
      }
    const float sc2 = oracle_bf16_round(1.5f);
    for (int64_t m = 0; m < M; ++m)
      for (int64_t n = 0; n < N; ++n) {
        double acc = 0;
        for (int64_t r = 0; r < R2; ++r) acc += (double)xa[m * R2 + r] * b2[r * N + n];
        const float res = oracle_bf16_round(oracle_bf16_round((float)acc) * sc2);
        ref[m * N + n] = oracle_bf16_round(ref[m * N + n] + res);
      }
    const double e = rel_fro(host_f32(y), ref);
    EXPECT(e < 2e-3, "relFro %.3e", e);
  }

  banner("AdaptableLinear promotion: f32 bias, bf16 then f32 LoRA factors; graph capture");
  {
    // A snapshot loaded as is keeps an f32 bias and f32 adapter factors (src/adapters.rs:243-252):
    // y0 bf16 + f32 bias -> f32, + bf16 adapter (residual bf16, sum f32), + f32 adapter -> f32.
    std::mt19937 rng(9);
    const int64_t M = 300, K = 512, N = 320, R1 = 16, R2 = 8;
    std::vector<float> w = bf16_normal(rng, N * K, 0.02f), x = bf16_normal(rng, M * K, 1.0f);
    std::vector<float> bias(N);
    std::normal_distribution<float> nd(0.0f, 0.3f);
    for (auto& v : bias) v = nd(rng);  // f32 values, not bf16-exact
    std::vector<float> a1 = bf16_normal(rng, K * R1, 0.02f), b1 = bf16_normal(rng, R1 * N, 0.02f);
    std::vector<float> a2(K * R2), b2(R2 * N);
    for (auto& v : a2) v = nd(rng) * 0.05f;
    for (auto& v : b2) v = nd(rng) * 0.05f;
    QuantizedLinear q = QuantizedLinear::try_from_linear(bf16_array(w, {N, K}),
                                                         Array::from_host(bias.data(), {N}, Dtype::Float32), 64, 4);
    AdaptableLinear l = AdaptableLinear::from_quantized_parts(q.weight, q.scales, q.biases, q.bias, 64, 4);
    l.push(Adapter{bf16_array(a1, {K, R1}), bf16_array(b1, {R1, N}), 0.5f});
    l.push(Adapter{Array::from_host(a2.data(), {K, R2}, Dtype::Float32),
                   Array::from_host(b2.data(), {R2, N}, Dtype::Float32), 1.25f});
    const Array xin = bf16_array(x, {M, K});
    EXPECT(l.out_dtype(Dtype::Bfloat16) == Dtype::Float32, "promoted dtype");
    Array y = l.forward(xin);
    EXPECT(y.dtype() == Dtype::Float32 && y.shape() == std::vector<int64_t>({M, N}), "promoted output");
    // reference: oracle linear with the f32 bias and adapter 1 (sum in f32), then adapter 2 in f32
    std::vector<uint32_t> wq(N * K / 8);
    std::vector<float> sc(N * K / 64), zz(N * K / 64), ref(M * N);
    oracle_quantize(w.data(), N, K, 64, 4, 1, wq.data(), sc.data(), zz.data());
    int ob = -1;
    oracle_linear(x.data(), M, K, wq.data(), sc.data(), zz.data(), N, 64, 4, 1, 1, 1, bias.data(), 0,
                  a1.data(), b1.data(), R1, 1, 0.5f, 0, ref.data(), &ob);
    EXPECT(ob == 0, "oracle dtype");
    for (int64_t m = 0; m < M; ++m) {
      double xa[R2];
      for (int64_t r = 0; r < R2; ++r) {
        double acc = 0;
        for (int64_t k = 0; k < K; ++k) acc += (double)x[m * K + k] * a2[k * R2 + r];
        xa[r] = (float)acc;
      }
      for (int64_t n = 0; n < N; ++n) {
        double acc = 0;
        for (int64_t r = 0; r < R2; ++r) acc += xa[r] * b2[r * N + n];
        ref[m * N + n] = (float)(ref[m * N + n] + (float)((float)acc * 1.25f));
      }
    }
    const std::vector<float> yh = host_f32(y);
    double e = rel_fro(yh, ref);
    EXPECT(e < 2e-3, "promoted relFro %.3e", e);
    // The same forward into a caller's array, captured in a HIP graph and replayed: the layer
    // allocates nothing and waits for nothing after its first call.
    hipStream_t st;
    EXPECT(hipStreamCreate(&st) == hipSuccess, "stream");
    Array out = Array::empty({M, N}, Dtype::Float32);
    l.forward_into(xin, out, st);  // first call: workspaces
    EXPECT(hipStreamSynchronize(st) == hipSuccess, "sync");
    EXPECT(host_f32(out) == yh, "forward_into differs from forward");
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    EXPECT(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal) == hipSuccess, "begin capture");
    l.forward_into(xin, out, st);
    EXPECT(hipStreamEndCapture(st, &graph) == hipSuccess, "end capture");
    EXPECT(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess, "instantiate");
    for (int rep = 0; rep < 3; ++rep) {
      EXPECT(hipMemsetAsync(out.data(), 0, out.nbytes(), st) == hipSuccess, "clear");
      EXPECT(hipGraphLaunch(exec, st) == hipSuccess, "replay");
      EXPECT(hipStreamSynchronize(st) == hipSuccess, "sync");
      EXPECT(host_f32(out) == yh, "graph replay %d differs from the eager result", rep);
      (void)l.forward(xin);  // eager work between replays
    }
    (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    (void)hipStreamDestroy(st);
  }

  banner("AdaptableLinear: LoKr adapters (bf16 LoRA + LoKr stack, LoKr first on an f32 stream, scale 0)");
  {
    std::mt19937 rng(13);
    const int64_t M = 150, K = 256, N = 200, R = 16;
    std::vector<float> w = bf16_normal(rng, N * K, 0.02f), xb = bf16_normal(rng, M * K, 1.0f);
    std::vector<float> a = bf16_normal(rng, K * R, 0.02f), b = bf16_normal(rng, R * N, 0.02f);
    std::vector<float> delta = bf16_normal(rng, N * K, 0.01f);  // stored bf16, as the reference does
    QuantizedLinear q = QuantizedLinear::try_from_linear(bf16_array(w, {N, K}), std::nullopt, 64, 4);
    std::vector<uint32_t> wq(N * K / 8);
    std::vector<float> sc(N * K / 64), zz(N * K / 64);
    oracle_quantize(w.data(), N, K, 64, 4, 1, wq.data(), sc.data(), zz.data());
    // bf16 x: base + LoRA (fused), then + LoKr (residual and sum in bf16)
    AdaptableLinear l = AdaptableLinear::from_quantized_parts(q.weight, q.scales, q.biases, std::nullopt, 64, 4);
    l.push(Adapter::lora(bf16_array(a, {K, R}), bf16_array(b, {R, N}), 0.5f));
    l.push(Adapter::lokr(bf16_array(delta, {N, K}), 0.7f));
    Array y = l.forward(bf16_array(xb, {M, K}));
    EXPECT(y.dtype() == Dtype::Bfloat16 && y.shape() == std::vector<int64_t>({M, N}), "lora+lokr output");
    std::vector<float> ref(M * N), ref2(M * N);
    oracle_linear(xb.data(), M, K, wq.data(), sc.data(), zz.data(), N, 64, 4, 1, 1, 1, nullptr, 1, a.data(),
                  b.data(), R, 1, 0.5f, 0, ref.data(), nullptr);
    int ob = -1;
    oracle_lokr_residual(xb.data(), M, K, delta.data(), N, 0.7f, 1, ref.data(), 1, ref2.data(), &ob);
    EXPECT(ob == 1, "oracle dtype");
    double e = rel_fro(host_f32(y), ref2);
    EXPECT(e < 2e-3, "lora+lokr relFro %.3e", e);
    // f32 x (FLUX.1's stream): LoKr first (nothing fused), the delta widened exactly, all in f32
    std::vector<float> xf(M * K);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (auto& v : xf) v = nd(rng);
    AdaptableLinear lf = AdaptableLinear::from_quantized_parts(q.weight, q.scales, q.biases, std::nullopt, 64, 4);
    lf.push(Adapter::lokr(bf16_array(delta, {N, K}), 1.25f));
    const Array xin = Array::from_host(xf.data(), {M, K}, Dtype::Float32);
    Array yf = lf.forward(xin);
    EXPECT(yf.dtype() == Dtype::Float32, "f32 stream output");
    oracle_linear(xf.data(), M, K, wq.data(), sc.data(), zz.data(), N, 64, 4, 0, 0, 1, nullptr, 1, nullptr,
                  nullptr, 0, 1, 1.0f, 0, ref.data(), nullptr);
    oracle_lokr_residual(xf.data(), M, K, delta.data(), N, 1.25f, 0, ref.data(), 0, ref2.data(), &ob);
    EXPECT(ob == 0, "oracle f32 dtype");
    e = rel_fro(host_f32(yf), ref2);
    EXPECT(e < 1e-4, "f32 lokr relFro %.3e", e);
    // scale 0 is a bit-exact no-op (src/adapters.rs:717-728)
    AdaptableLinear l0 = AdaptableLinear::from_quantized_parts(q.weight, q.scales, q.biases, std::nullopt, 64, 4);
    const Array base = l0.forward(xin);
    l0.push(Adapter::lokr(bf16_array(delta, {N, K}), 0.0f));
    EXPECT(host_f32(l0.forward(xin)) == host_f32(base), "scale-0 LoKr changed the output");
    // a wrongly shaped delta is an error, not a crash
    l0.push(Adapter::lokr(bf16_array(delta, {K, N}), 1.0f));
    bool threw = false;
    try { l0.forward(xin); } catch (const Error& err) { threw = err.status == MLXQ_EINVAL; }
    EXPECT(threw, "a [in, out] delta accepted");
  }

  banner("fused SwiGLU decode and the stacked expert projection");
  {
    std::mt19937 rng(21);
    const int64_t K = 512, F = 192, M = 3;
    std::vector<float> wg = bf16_normal(rng, F * K, 0.02f), wu = bf16_normal(rng, F * K, 0.02f);
    std::vector<float> xv = bf16_normal(rng, M * K, 1.0f);
    QuantizedLinear gate = QuantizedLinear::try_from_linear(bf16_array(wg, {F, K}), std::nullopt, 64, 4);
    QuantizedLinear up = QuantizedLinear::try_from_linear(bf16_array(wu, {F, K}), std::nullopt, 64, 4);
    Array h = swiglu(bf16_array(xv, {M, K}), gate, up);
    EXPECT(h.shape() == std::vector<int64_t>({M, F}) && h.dtype() == Dtype::Bfloat16, "swiglu shape");
    std::vector<uint32_t> qg(F * K / 8), qu(F * K / 8);
    std::vector<float> sg(F * K / 64), zg(F * K / 64), su(F * K / 64), zu(F * K / 64), g(M * F), u(M * F);
    oracle_quantize(wg.data(), F, K, 64, 4, 1, qg.data(), sg.data(), zg.data());
    oracle_quantize(wu.data(), F, K, 64, 4, 1, qu.data(), su.data(), zu.data());
    oracle_qmm(xv.data(), M, K, qg.data(), sg.data(), zg.data(), F, 64, 4, 0, 1, g.data());
    oracle_qmm(xv.data(), M, K, qu.data(), su.data(), zu.data(), F, 64, 4, 0, 1, u.data());
    std::vector<float> ref(M * F);
    for (int64_t i = 0; i < M * F; ++i) ref[i] = oracle_bf16_round(oracle_silu(g[i], 1) * u[i]);
    double e = rel_fro(host_f32(h), ref);
    EXPECT(e < 2e-3, "swiglu relFro %.3e", e);
    bool unsupported = false;
    try { swiglu(bf16_array(bf16_normal(rng, 20 * K, 1.0f), {20, K}), gate, up); }
    catch (const Error& err) { unsupported = err.status == MLXQ_EUNSUPPORTED; }
    EXPECT(unsupported, "swiglu outside the decode form reports EUNSUPPORTED");

    // Experts: pack the stack [E*N, K] in one call, run every expert, compare with the split layers.
    const int64_t E = 4, N = 96, Ke = 256, Mt = 40;
    std::vector<float> we = bf16_normal(rng, E * N * Ke, 0.02f), be = bf16_normal(rng, E * N, 0.5f);
    Packed p = quantize(bf16_array(we, {E * N, Ke}), 64, 4);
    StackedExperts st{p.wq.reshape({E, N, Ke / 8}), p.scales.reshape({E, N, Ke / 64}),
                      p.biases.reshape({E, N, Ke / 64}), bf16_array(be, {E, N}), 64, 4};
    std::vector<float> xs = bf16_normal(rng, Mt * Ke, 1.0f);
    Array y = st.forward(bf16_array(xs, {Mt, Ke}));
    EXPECT(y.shape() == std::vector<int64_t>({E, Mt, N}), "experts shape");
    std::vector<float> yh = host_f32(y);
    std::vector<QuantizedLinear> parts = st.split();
    for (int64_t ex = 0; ex < E; ++ex) {
      std::vector<float> one = host_f32(parts[ex].forward(bf16_array(xs, {Mt, Ke})));
      std::vector<float> mine(yh.begin() + ex * Mt * N, yh.begin() + (ex + 1) * Mt * N);
      e = rel_fro(mine, one);
      EXPECT(e < 2e-3, "expert %lld relFro %.3e", (long long)ex, e);
    }
    // Odd N with one group per row (K = 64) and M = 3: every expert's y and scales slices are
    // unaligned for the expert-by-expert launches, so the host runs them on aligned copies.
    const int64_t No = 37, Ko = 64, Mo = 3;
    std::vector<float> wo = bf16_normal(rng, E * No * Ko, 0.02f), bo = bf16_normal(rng, E * No, 0.5f);
    Packed po = quantize(bf16_array(wo, {E * No, Ko}), 64, 4);
    StackedExperts so{po.wq.reshape({E, No, Ko / 8}), po.scales.reshape({E, No, 1}),
                      po.biases.reshape({E, No, 1}), bf16_array(bo, {E, No}), 64, 4};
    std::vector<float> xo = bf16_normal(rng, Mo * Ko, 1.0f);
    std::vector<float> yo = host_f32(so.forward(bf16_array(xo, {Mo, Ko})));
    std::vector<QuantizedLinear> po_parts = so.split();
    for (int64_t ex = 0; ex < E; ++ex) {
      std::vector<float> one = host_f32(po_parts[ex].forward(bf16_array(xo, {Mo, Ko})));
      std::vector<float> mine(yo.begin() + ex * Mo * No, yo.begin() + (ex + 1) * Mo * No);
      EXPECT(mine == one, "unaligned expert %lld differs from its own layer", (long long)ex);
    }
  }

  banner("TokenEmbedding quantize + forward, and the snapshot round trip");
  {
    std::mt19937 rng(11);
    const int64_t vocab = 300, hidden = 128;
    std::vector<float> table = bf16_normal(rng, vocab * hidden, 0.02f);
    TokenEmbedding e = TokenEmbedding::dense(bf16_array(table, {vocab, hidden}));
    e.quantize(8, true);
    std::vector<int32_t> ids = {0, 299, 5, 5, 123, 42};
    Array out = e.forward(Array::from_host(ids.data(), {2, 3}, Dtype::Int32));
    EXPECT(out.shape() == std::vector<int64_t>({2, 3, hidden}) && out.dtype() == Dtype::Float32, "shape");
    std::vector<uint32_t> wq(vocab * hidden / 4);
    std::vector<float> s(vocab * hidden / 64), z(vocab * hidden / 64), deq(vocab * hidden);
    oracle_quantize(table.data(), vocab, hidden, 64, 8, 1, wq.data(), s.data(), z.data());
    oracle_dequantize(wq.data(), s.data(), z.data(), vocab, hidden, 64, 8, 1, deq.data());
    auto got = host<float>(out);
    bool same = true;
    for (size_t t = 0; t < ids.size(); ++t)
      same &= memcmp(&got[t * hidden], &deq[ids[t] * hidden], hidden * 4) == 0;
    EXPECT(same, "embedding rows differ from dequantize");

    // quantize_map -> save_map -> load_dir_map -> lin / embedding
    const fs::path dir = fs::temp_directory_path() / ("mlxq_snap_" + std::to_string(::getpid()));
    Weights m;
    std::vector<float> wlin = bf16_normal(rng, 96 * 256, 0.02f);
    m["blk.q.weight"] = bf16_array(wlin, {96, 256});
    m["blk.norm.weight"] = bf16_array(std::vector<float>(256, 1.0f), {256});
    m["embed.weight"] = bf16_array(table, {vocab, hidden});
    Weights packed = quantize_map(m, 4, 32, [](const std::string& b) { return b != "blk.norm"; });
    EXPECT(packed.count("blk.q.scales") && packed.count("embed.biases") && !packed.count("blk.norm.scales"),
           "quantize_map keys");
    {  // two targets of one shape: packed in one batched launch, the same triples as quantize()
      Weights m2;
      std::vector<float> wa = bf16_normal(rng, 64 * 128, 0.02f), wb = bf16_normal(rng, 64 * 128, 0.05f);
      m2["a.weight"] = bf16_array(wa, {64, 128});
      m2["b.weight"] = bf16_array(wb, {64, 128});
      Weights p2 = quantize_map(m2, 8, 64, [](const std::string&) { return true; });
      for (const char* base : {"a", "b"}) {
        Packed one = quantize(m2.at(std::string(base) + ".weight"), 64, 8);
        EXPECT(host<uint32_t>(p2.at(std::string(base) + ".weight")) == host<uint32_t>(one.wq) &&
                   host<uint16_t>(p2.at(std::string(base) + ".scales")) == host<uint16_t>(one.scales) &&
                   host<uint16_t>(p2.at(std::string(base) + ".biases")) == host<uint16_t>(one.biases),
               "batched quantize_map differs from quantize");
      }
    }
    save_map((dir / "model.safetensors").string(), packed);
    HostMap raw = read_safetensors((dir / "model.safetensors").string());
    EXPECT(raw.at("blk.q.weight").dtype == Dtype::Uint32, "codes stored as U32");
    Weights back = load_dir_map(dir.string());
    AdaptableLinear q = lin(back, "blk.q", false, 32);
    EXPECT(q.is_quantized() && q.quantized().bits == 4, "lin packed");
    EXPECT(!lin(back, "blk.norm", false, 32).is_quantized(), "lin dense");
    TokenEmbedding te = embedding(back, "embed", 32);
    EXPECT(te.is_quantized() && te.bits() == 4 && te.group_size() == 32, "embedding packed");
    std::vector<float> xq = bf16_normal(rng, 3 * 256, 1.0f);
    auto y1 = host_f32(q.forward(bf16_array(xq, {3, 256})));
    AdaptableLinear orig = AdaptableLinear::from_quantized_parts(
        packed["blk.q.weight"], packed["blk.q.scales"], packed["blk.q.biases"], std::nullopt, 32, 4);
    auto y2 = host_f32(orig.forward(bf16_array(xq, {3, 256})));
    EXPECT(y1 == y2, "reloaded linear differs");
    fs::remove_all(dir);
  }
}

int main(int argc, char** argv) {
  if (argc < 2 || (strcmp(argv[1], "cpu") && strcmp(argv[1], "gpu"))) {
    fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  const fs::path root = repo_root(argv[0]);
  try {
    if (!strcmp(argv[1], "cpu")) cpu_cases(root);
    else gpu_cases(root);
  } catch (const std::exception& e) {
    fprintf(stderr, "FAIL: uncaught exception: %s\n", e.what());
    return 1;
  }
  if (g_failures) {
    fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  printf("ALL PASS (%s)\n", argv[1]);
  return 0;
}
