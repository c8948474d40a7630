// host.cpp — Array, the op triple and the layer types of the C++ host API (see mlxq.hpp).
// Every computation goes through the C ABI of libmlxq_hip.so; this file only allocates device
// memory, checks shapes the way the reference's callers rely on, and sequences ABI calls.
#include "mlxq.hpp"

#include <cstring>

#include "../../include/mlxq.h"

namespace mlxq {

namespace {

void check(int status) {
  if (status != MLXQ_OK) throw Error(status, mlxq_last_error());
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(MLXQ_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// The ABI code of a float dtype.  float16 is taken by the ABI as activations only; where an entry
// point does not take it, the library reports MLXQ_EUNSUPPORTED.
int abi_dtype(Dtype dt, const char* op) {
  if (dt == Dtype::Float32) return MLXQ_FLOAT32;
  if (dt == Dtype::Bfloat16) return MLXQ_BFLOAT16;
  if (dt == Dtype::Float16) return MLXQ_FLOAT16;
  throw Error(MLXQ_EINVAL, std::string(op) + ": expected a float32, bfloat16 or float16 array, got " +
                               dtype_name(dt));
}

void need_packed(const Array& wq, const char* op) {
  if (wq.dtype() != Dtype::Uint32 && wq.dtype() != Dtype::Int32)
    throw Error(MLXQ_EINVAL, std::string(op) + ": packed weights must be uint32");
  if (wq.ndim() != 2) throw Error(MLXQ_EINVAL, std::string(op) + ": packed weights must be 2-D");
}

Dtype from_abi(int dt) {
  return dt == MLXQ_BFLOAT16 ? Dtype::Bfloat16 : dt == MLXQ_FLOAT16 ? Dtype::Float16 : Dtype::Float32;
}

// MLX's result type over float operands: a 16-bit type only when both have it; f32 otherwise
// (bf16 meeting fp16 included).
Dtype promote(Dtype a, Dtype b) {
  if (a == b && (a == Dtype::Bfloat16 || a == Dtype::Float16)) return a;
  return Dtype::Float32;
}

// The packed triple against x's width K, as MLX's quantized_matmul checks it
// (extract_quantized_matmul_dims): wq [..., N, K*bits/32], scales/biases [..., N, K/gs] alike.
// `lead` leading dimensions (the expert axis of a stack) must match too.  Returns N.
int64_t check_pack(const char* op, const Array& wq, const Array& scales, const Array& biases,
                   int64_t K, int group_size, int bits, int lead = 0) {
  const std::string o(op);
  if (bits != 4 && bits != 8) throw Error(MLXQ_EINVAL, o + ": bits must be 4 or 8");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    throw Error(MLXQ_EINVAL, o + ": group_size must be 32, 64 or 128");
  if (wq.dtype() != Dtype::Uint32 && wq.dtype() != Dtype::Int32)
    throw Error(MLXQ_EINVAL, o + ": packed weights must be uint32");
  const int nd = lead + 2;
  if (wq.ndim() != nd || scales.ndim() != nd || biases.ndim() != nd)
    throw Error(MLXQ_EINVAL, o + ": wq, scales and biases must be " + std::to_string(nd) + "-D");
  for (int i = 0; i < lead; ++i)
    if (scales.dim(i) != wq.dim(i) || biases.dim(i) != wq.dim(i))
      throw Error(MLXQ_EINVAL, o + ": stacked operands disagree on their leading dimensions");
  const int64_t N = wq.dim(lead);
  if (K % group_size != 0) throw Error(MLXQ_EINVAL, o + ": K is not a multiple of group_size");
  if (wq.dim(lead + 1) * 32 != K * bits)
    throw Error(MLXQ_EINVAL, o + ": wq has " + std::to_string(wq.dim(lead + 1)) +
                                 " words per row, which does not pack x's K=" + std::to_string(K));
  if (scales.dim(lead) != N || scales.dim(lead + 1) != K / group_size || biases.shape() != scales.shape())
    throw Error(MLXQ_EINVAL, o + ": scales/biases must be [N, K/group_size]");
  abi_dtype(scales.dtype(), op);
  if (biases.dtype() != scales.dtype()) throw Error(MLXQ_EINVAL, o + ": biases and scales dtypes differ");
  return N;
}

// The layer's reusable workspace grown to `need` bytes (empty array when none is needed).  It
// stays allocated with the layer, so forward calls after the first allocate nothing.
Array& grow_workspace(std::shared_ptr<Array>& ws, size_t need) {
  if (!ws) ws = std::make_shared<Array>();
  if (ws->nbytes() < need) *ws = Array::empty({(int64_t)((need + 3) / 4)}, Dtype::Uint32);
  return *ws;
}

}  // namespace

size_t dtype_size(Dtype dt) {
  switch (dt) {
    case Dtype::Float32: case Dtype::Uint32: case Dtype::Int32: return 4;
    case Dtype::Bfloat16: case Dtype::Float16: return 2;
    case Dtype::Int64: case Dtype::Float64: return 8;
    case Dtype::Uint8: case Dtype::Int8: case Dtype::Bool: return 1;
  }
  return 0;
}

const char* dtype_name(Dtype dt) {
  switch (dt) {
    case Dtype::Float32: return "F32";
    case Dtype::Bfloat16: return "BF16";
    case Dtype::Uint32: return "U32";
    case Dtype::Int32: return "I32";
    case Dtype::Float16: return "F16";
    case Dtype::Int64: return "I64";
    case Dtype::Uint8: return "U8";
    case Dtype::Int8: return "I8";
    case Dtype::Float64: return "F64";
    case Dtype::Bool: return "BOOL";
  }
  return "?";
}

Dtype dtype_from_name(const std::string& n) {
  static const std::pair<const char*, Dtype> table[] = {
      {"F32", Dtype::Float32}, {"BF16", Dtype::Bfloat16}, {"U32", Dtype::Uint32},
      {"I32", Dtype::Int32},   {"F16", Dtype::Float16},   {"I64", Dtype::Int64},
      {"U8", Dtype::Uint8},    {"I8", Dtype::Int8},       {"F64", Dtype::Float64},
      {"BOOL", Dtype::Bool}};
  for (const auto& e : table)
    if (n == e.first) return e.second;
  throw Error(MLXQ_EUNSUPPORTED, "unsupported tensor dtype " + n);
}

// ---- Array ------------------------------------------------------------------------------------

int64_t Array::size() const {
  int64_t n = 1;
  for (int64_t d : shape_) n *= d;
  return n;
}

Array Array::empty(std::vector<int64_t> shape, Dtype dt) {
  Array a;
  a.shape_ = std::move(shape);
  a.dtype_ = dt;
  for (int64_t d : a.shape_)
    if (d < 0) throw Error(MLXQ_EINVAL, "Array: negative dimension");
  if (a.nbytes() > 0) {
    void* p = nullptr;
    hip_check(hipMalloc(&p, a.nbytes()), "hipMalloc");
    a.buf_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
    a.ptr_ = p;
  }
  return a;
}

std::pair<Array, Array> Array::empty_pair(std::vector<int64_t> shape, Dtype dt) {
  Array a, b;
  a.shape_ = b.shape_ = std::move(shape);
  a.dtype_ = b.dtype_ = dt;
  for (int64_t d : a.shape_)
    if (d < 0) throw Error(MLXQ_EINVAL, "Array: negative dimension");
  const size_t n = a.nbytes();
  if (n > 0) {
    const size_t off = (n + 511) / 256 * 256;
    void* p = nullptr;
    hip_check(hipMalloc(&p, off + n), "hipMalloc");
    a.buf_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
    b.buf_ = a.buf_;
    a.ptr_ = p;
    b.ptr_ = static_cast<unsigned char*>(p) + off;
  }
  return {a, b};
}

Array Array::from_host(const void* data, std::vector<int64_t> shape, Dtype dt) {
  Array a = empty(std::move(shape), dt);
  if (a.nbytes() > 0) hip_check(hipMemcpy(a.ptr_, data, a.nbytes(), hipMemcpyHostToDevice), "hipMemcpy");
  return a;
}

Array Array::borrow(void* device_ptr, std::vector<int64_t> shape, Dtype dt) {
  Array a;
  a.shape_ = std::move(shape);
  a.dtype_ = dt;
  a.ptr_ = device_ptr;
  return a;
}

void Array::to_host(void* dst) const {
  if (nbytes() == 0) return;
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  hip_check(hipMemcpy(dst, ptr_, nbytes(), hipMemcpyDeviceToHost), "hipMemcpy");
}

Array Array::reshape(std::vector<int64_t> shape) const {
  Array a = *this;
  a.shape_ = std::move(shape);
  if (a.size() != size()) throw Error(MLXQ_EINVAL, "reshape: element count changes");
  return a;
}

Array Array::index0(int64_t i) const {
  if (ndim() < 1 || i < 0 || i >= shape_[0]) throw Error(MLXQ_EINVAL, "index0: index out of range");
  Array a = *this;
  a.shape_.erase(a.shape_.begin());
  a.ptr_ = a.size() > 0 ? (char*)ptr_ + (size_t)i * a.nbytes() : nullptr;
  return a;
}

// ---- ops --------------------------------------------------------------------------------------

Array as_dtype(const Array& a, Dtype dt, hipStream_t s) {
  if (a.dtype() == dt) return a;
  const int src = abi_dtype(a.dtype(), "as_dtype"), dst = abi_dtype(dt, "as_dtype");
  Array out = Array::empty(a.shape(), dt);
  check(mlxq_cast(a.data(), src, out.data(), dst, a.size(), s));
  return out;
}

Packed quantize(const Array& w, int group_size, int bits, hipStream_t s) {
  if (w.ndim() != 2) throw Error(MLXQ_EINVAL, "quantize: expected a 2-D weight");
  const int dt = abi_dtype(w.dtype(), "quantize");
  const int64_t N = w.dim(0), K = w.dim(1);
  const int64_t gcols = group_size > 0 ? K / group_size : 0;
  auto sb = Array::empty_pair({N, gcols}, w.dtype());
  Packed p{Array::empty({N, bits > 0 ? K * bits / 32 : 0}, Dtype::Uint32), sb.first, sb.second};
  check(mlxq_quantize(w.data(), dt, N, K, group_size, bits, (uint32_t*)p.wq.data(), p.scales.data(),
                      p.biases.data(), s));
  return p;
}

std::vector<Packed> quantize_batched(const std::vector<Array>& ws, int group_size, int bits, hipStream_t s) {
  std::vector<Packed> out;
  if (ws.empty()) return out;
  const Array& w0 = ws[0];
  if (w0.ndim() != 2) throw Error(MLXQ_EINVAL, "quantize_batched: expected 2-D weights");
  for (const Array& w : ws)
    if (w.shape() != w0.shape() || w.dtype() != w0.dtype())
      throw Error(MLXQ_EINVAL, "quantize_batched: every weight must have the first one's shape and dtype");
  const int dt = abi_dtype(w0.dtype(), "quantize_batched");
  const int64_t N = w0.dim(0), K = w0.dim(1);
  const int64_t gcols = group_size > 0 ? K / group_size : 0;
  std::vector<const void*> wp;
  std::vector<uint32_t*> qp;
  std::vector<void*> sp, bp;
  for (const Array& w : ws) {
    auto sb = Array::empty_pair({N, gcols}, w0.dtype());
    out.push_back(Packed{Array::empty({N, bits > 0 ? K * bits / 32 : 0}, Dtype::Uint32), sb.first, sb.second});
    wp.push_back(w.data());
    qp.push_back((uint32_t*)out.back().wq.data());
    sp.push_back(out.back().scales.data());
    bp.push_back(out.back().biases.data());
  }
  check(mlxq_quantize_batched(wp.data(), (int)ws.size(), dt, N, K, group_size, bits, qp.data(), sp.data(),
                              bp.data(), s));
  return out;
}

Array dequantize(const Array& wq, const Array& scales, const Array& biases, int group_size, int bits,
                 hipStream_t s) {
  need_packed(wq, "dequantize");
  if (bits != 4 && bits != 8) throw Error(MLXQ_EINVAL, "dequantize: bits must be 4 or 8");
  const int64_t K = wq.dim(1) * 32 / bits;
  const int64_t N = check_pack("dequantize", wq, scales, biases, K, group_size, bits);
  Array out = Array::empty({N, K}, scales.dtype());
  check(mlxq_dequantize((const uint32_t*)wq.data(), scales.data(), biases.data(),
                        abi_dtype(scales.dtype(), "dequantize"), N, K, group_size, bits, out.data(), s));
  return out;
}

Array quantized_matmul(const Array& x, const Array& wq, const Array& scales, const Array& biases,
                       bool transpose, int group_size, int bits, hipStream_t s) {
  need_packed(wq, "quantized_matmul");
  if (x.ndim() < 1) throw Error(MLXQ_EINVAL, "quantized_matmul: x must have a last dimension");
  abi_dtype(x.dtype(), "quantized_matmul");
  const int64_t K = x.dim(-1), M = K > 0 ? x.size() / K : 0;
  const int64_t N = check_pack("quantized_matmul", wq, scales, biases, K, group_size, bits);
  std::vector<int64_t> shape = x.shape();
  shape.back() = N;
  Array y = Array::empty(shape, promote(x.dtype(), scales.dtype()));
  check(mlxq_quantized_matmul(x.data(), abi_dtype(x.dtype(), "quantized_matmul"), M, K,
                              (const uint32_t*)wq.data(), scales.data(), biases.data(),
                              abi_dtype(scales.dtype(), "quantized_matmul"), N, transpose ? 1 : 0,
                              group_size, bits, y.data(), s));
  return y;
}

int packed_bits(const Array& wq, const Array& scales, int group_size) {
  if (wq.ndim() != 2 || scales.ndim() != 2) throw Error(MLXQ_EINVAL, "packed_bits: expected 2-D arrays");
  const int b = mlxq_packed_bits(wq.dim(1), scales.dim(1), group_size);
  if (b < 0) throw Error(MLXQ_EINVAL, mlxq_last_error());
  return b;
}

Array swiglu(const Array& x, const QuantizedLinear& gate, const QuantizedLinear& up, hipStream_t s) {
  need_packed(gate.weight, "swiglu");
  need_packed(up.weight, "swiglu");
  if (gate.bias || up.bias) throw Error(MLXQ_EUNSUPPORTED, "swiglu: projections with a dense bias");
  if (gate.group_size != up.group_size || gate.bits != up.bits ||
      gate.weight.shape() != up.weight.shape() || x.ndim() < 1 || x.dim(-1) != gate.in_features() ||
      gate.scales.dtype() != up.scales.dtype())
    throw Error(MLXQ_EINVAL, "swiglu: gate and up must be packed alike and match x");
  const int64_t K = x.dim(-1), M = K > 0 ? x.size() / K : 0;
  const int64_t F = check_pack("swiglu", gate.weight, gate.scales, gate.biases, K, gate.group_size, gate.bits);
  check_pack("swiglu", up.weight, up.scales, up.biases, K, up.group_size, up.bits);
  std::vector<int64_t> shape = x.shape();
  shape.back() = F;
  Array h = Array::empty(shape, promote(x.dtype(), gate.scales.dtype()));
  check(mlxq_swiglu(x.data(), abi_dtype(x.dtype(), "swiglu"), M, K,
                    (const uint32_t*)gate.weight.data(), gate.scales.data(), gate.biases.data(),
                    (const uint32_t*)up.weight.data(), up.scales.data(), up.biases.data(),
                    abi_dtype(gate.scales.dtype(), "swiglu"), F, gate.group_size, gate.bits, h.data(), s));
  return h;
}

std::vector<QuantizedLinear> StackedExperts::split() const {
  // Views of the stack, as the reference's split; an expert's scales/biases slice that does not
  // start on a 4-byte boundary (N * K/group_size odd in bf16) is copied instead, since the library
  // reads scales and biases as whole words.
  const int64_t E = num_experts();
  const bool copy_sb = E > 0 && (scales.nbytes() / (size_t)E) % 4 != 0;
  auto copy_of = [](const Array& a) {
    Array c = Array::empty(a.shape(), a.dtype());
    if (c.nbytes() > 0) hip_check(hipMemcpy(c.data(), a.data(), c.nbytes(), hipMemcpyDeviceToDevice), "hipMemcpy");
    return c;
  };
  std::vector<QuantizedLinear> out;
  for (int64_t e = 0; e < E; ++e)
    out.push_back(QuantizedLinear{weight.index0(e), copy_sb ? copy_of(scales.index0(e)) : scales.index0(e),
                                  copy_sb ? copy_of(biases.index0(e)) : biases.index0(e),
                                  bias ? std::optional<Array>(bias->index0(e)) : std::nullopt,
                                  group_size, bits});
  return out;
}

Array StackedExperts::forward(const Array& x, bool per_expert, hipStream_t s) const {
  if (weight.dtype() != Dtype::Uint32 && weight.dtype() != Dtype::Int32)
    throw Error(MLXQ_EINVAL, "experts: weight must hold packed uint32 codes");
  if (weight.ndim() != 3 || scales.ndim() != 3 || x.ndim() < 1)
    throw Error(MLXQ_EINVAL, "experts: expected [E, out, ...] stacks");
  const int64_t E = num_experts(), K = x.dim(-1);
  const int64_t N = check_pack("experts", weight, scales, biases, K, group_size, bits, 1);
  if (bias && (bias->ndim() != 2 || bias->dim(0) != E || bias->dim(1) != N))
    throw Error(MLXQ_EINVAL, "experts: bias must be [E, out]");
  std::vector<int64_t> lead(x.shape().begin() + (per_expert ? 1 : 0), x.shape().end() - 1);
  if (per_expert && (x.ndim() < 2 || x.dim(0) != E))
    throw Error(MLXQ_EINVAL, "experts: per-expert x must lead with E");
  int64_t M = 1;
  for (int64_t d : lead) M *= d;
  std::vector<int64_t> shape = {E};
  shape.insert(shape.end(), lead.begin(), lead.end());
  shape.push_back(N);
  Dtype ydt = promote(x.dtype(), scales.dtype());
  if (bias) ydt = promote(ydt, bias->dtype());
  Array y = Array::empty(shape, ydt);
  const int xdt = abi_dtype(x.dtype(), "experts"), sdt = abi_dtype(scales.dtype(), "experts");
  const int bdt = bias ? abi_dtype(bias->dtype(), "experts") : MLXQ_BFLOAT16;
  const int rc = mlxq_qmm_experts(x.data(), xdt, per_expert ? 1 : 0, E, M, K, (const uint32_t*)weight.data(),
                                  scales.data(), biases.data(), sdt, bias ? bias->data() : nullptr, bdt, N,
                                  group_size, bits, y.data(), s);
  const size_t ysz = dtype_size(ydt), ssz = dtype_size(scales.dtype());
  const int64_t G = K / group_size;
  const bool misaligned = E > 1 && ((M * N * (int64_t)ysz) % 16 != 0 || (N * G * (int64_t)ssz) % 4 != 0);
  if (rc != MLXQ_EUNSUPPORTED || !misaligned) {
    check(rc);
    return y;
  }
  // The library runs these experts one at a time and an expert's slice of y or of the
  // scales/biases is unaligned for it: run them here on aligned copies.
  const size_t xsz = dtype_size(x.dtype());
  Array se = Array::empty({N, G}, scales.dtype()), be = Array::empty({N, G}, scales.dtype());
  Array ye = Array::empty({M, N}, ydt);
  for (int64_t e = 0; e < E; ++e) {
    hip_check(hipMemcpyAsync(se.data(), static_cast<const char*>(scales.data()) + e * N * G * ssz, se.nbytes(),
                             hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
    hip_check(hipMemcpyAsync(be.data(), static_cast<const char*>(biases.data()) + e * N * G * ssz, be.nbytes(),
                             hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
    mlxq_epilogue ep = {};
    ep.lora_scale = 1.0f;
    ep.bias_dtype = bias ? bdt : xdt;
    ep.lora_dtype = xdt;
    if (bias) ep.bias = static_cast<const char*>(bias->data()) + e * N * dtype_size(bias->dtype());
    check(mlxq_linear(static_cast<const char*>(x.data()) + (per_expert ? e * M * K * xsz : 0), xdt, M, K,
                      static_cast<const uint32_t*>(weight.data()) + e * N * (K * bits / 32), se.data(), be.data(),
                      sdt, N, group_size, bits, &ep, ye.data(), nullptr, 0, s));
    hip_check(hipMemcpyAsync(static_cast<char*>(y.data()) + e * M * N * ysz, ye.data(), ye.nbytes(),
                             hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
  }
  return y;
}

// ---- layers -----------------------------------------------------------------------------------

QuantizedLinear QuantizedLinear::try_from_linear(const Array& weight, std::optional<Array> bias,
                                                 int group_size, int bits, hipStream_t s) {
  Packed p = quantize(weight, group_size, bits, s);
  return QuantizedLinear{p.wq, p.scales, p.biases, std::move(bias), group_size, bits};
}

Array QuantizedLinear::forward(const Array& x, hipStream_t s) const {
  return forward_fused(x, nullptr, MLXQ_ACT_NONE, s);
}

namespace {
// `out` when given (checked against the result's shape and dtype), else a new array.
Array output_array(const Array* out, const std::vector<int64_t>& shape, Dtype dt, const char* op) {
  if (!out) return Array::empty(shape, dt);
  if (out->shape() != shape || out->dtype() != dt)
    throw Error(MLXQ_EINVAL, std::string(op) + ": out has the wrong shape or dtype (want " +
                                 dtype_name(dt) + ")");
  return *out;
}
}  // namespace

Array QuantizedLinear::forward_fused(const Array& x, const Adapter* lora, int activation,
                                     hipStream_t s, const Array* out) const {
  // src/adapters.rs:309-320,543-549: quantized_matmul, then the dense bias and the adapter's
  // residual as separate adds, each in its promoted dtype (bias and factors keep theirs).
  if (x.ndim() < 1) throw Error(MLXQ_EINVAL, "linear: x must have a last dimension");
  const int xdt = abi_dtype(x.dtype(), "linear");
  const int64_t K = x.dim(-1), M = K > 0 ? x.size() / K : 0;
  const int64_t N = check_pack("linear", weight, scales, biases, K, group_size, bits);
  mlxq_epilogue e = {};
  e.lora_scale = 1.0f;
  e.activation = activation;
  e.bias_dtype = e.lora_dtype = xdt;
  if (bias) {
    if (bias->ndim() != 1 || bias->dim(0) != N) throw Error(MLXQ_EINVAL, "linear: bias must be [out]");
    e.bias = bias->data();
    e.bias_dtype = abi_dtype(bias->dtype(), "linear");
  }
  if (lora) {
    if (lora->a.ndim() != 2 || lora->b.ndim() != 2 || lora->a.dim(0) != K || lora->b.dim(1) != N ||
        lora->a.dim(1) != lora->b.dim(0) || lora->a.dtype() != lora->b.dtype())
      throw Error(MLXQ_EINVAL, "linear: LoRA factors must be A [in, r] and B [r, out] of one dtype");
    e.lora_a = lora->a.data();
    e.lora_b = lora->b.data();
    e.lora_rank = lora->a.dim(1);
    e.lora_scale = lora->scale;
    e.lora_dtype = abi_dtype(lora->a.dtype(), "linear");
  }
  const int sdt = abi_dtype(scales.dtype(), "linear");
  const int ydt = mlxq_linear_out_dtype(xdt, sdt, &e);
  if (ydt < 0) throw Error(MLXQ_EINVAL, mlxq_last_error());
  std::vector<int64_t> shape = x.shape();
  shape.back() = N;
  Array y = output_array(out, shape, from_abi(ydt), "linear");
  Array& ws = grow_workspace(workspace_, mlxq_linear_workspace_size(xdt, sdt, M, N, &e));
  check(mlxq_linear(x.data(), xdt, M, K, (const uint32_t*)weight.data(), scales.data(), biases.data(),
                    sdt, N, group_size, bits, &e, y.data(), ws.nbytes() ? ws.data() : nullptr,
                    ws.nbytes(), s));
  return y;
}

AdaptableLinear AdaptableLinear::dense(Array weight, std::optional<Array> bias) {
  AdaptableLinear l;
  l.dense_weight_ = std::move(weight);
  l.dense_bias_ = std::move(bias);
  return l;
}

AdaptableLinear AdaptableLinear::from_quantized_parts(Array weight, Array scales, Array biases,
                                                      std::optional<Array> bias, int group_size,
                                                      int bits) {
  AdaptableLinear l;
  l.quantized_ = QuantizedLinear{std::move(weight), std::move(scales), std::move(biases), std::move(bias),
                                 group_size, bits};
  return l;
}

std::array<int64_t, 2> AdaptableLinear::base_shape() const {
  if (quantized_) return {quantized_->scales.dim(0), quantized_->in_features()};
  return {dense_weight_->dim(0), dense_weight_->dim(1)};
}

void AdaptableLinear::quantize(int bits, std::optional<int> group_size, hipStream_t s) {
  if (quantized_) return;
  const Array w = as_dtype(*dense_weight_, Dtype::Bfloat16, s);
  std::optional<Array> b;
  if (dense_bias_) b = as_dtype(*dense_bias_, Dtype::Bfloat16, s);
  quantized_ = QuantizedLinear::try_from_linear(w, b, group_size.value_or(64), bits, s);
  dense_weight_.reset();
  dense_bias_.reset();
}

Array AdaptableLinear::forward(const Array& x, hipStream_t s) const { return forward_impl(x, nullptr, s); }

void AdaptableLinear::forward_into(const Array& x, const Array& out, hipStream_t s) const {
  forward_impl(x, &out, s);
}

Dtype AdaptableLinear::out_dtype(Dtype x_dtype) const {
  if (!quantized_) throw Error(MLXQ_EUNSUPPORTED, "AdaptableLinear: the dense base is not on the quantized path");
  const QuantizedLinear& q = *quantized_;
  Dtype d = promote(x_dtype, q.scales.dtype());
  if (q.bias) d = promote(d, q.bias->dtype());
  for (const Adapter& ad : adapters_) d = promote(d, ad.is_lokr() ? x_dtype : promote(x_dtype, ad.a.dtype()));
  return d;
}

Array AdaptableLinear::forward_impl(const Array& x, const Array* out_arg, hipStream_t s) const {
  if (!quantized_)
    throw Error(MLXQ_EUNSUPPORTED,
                "AdaptableLinear: the dense base is not on the quantized path; call quantize() first");
  const QuantizedLinear& q = *quantized_;
  for (const Adapter& ad : adapters_)
    if (!ad.is_lokr() && (ad.a.ndim() != 2 || ad.a.dim(1) > 256))
      throw Error(MLXQ_EUNSUPPORTED, "AdaptableLinear: LoRA rank above 256");
  if (adapters_.empty()) return q.forward_fused(x, nullptr, MLXQ_ACT_NONE, s, out_arg);
  // A leading LoRA adapter rides in mlxq_linear's epilogue, the others are added one at a time
  // (out = out + residual, src/adapters.rs:545-547), each sum in MLX's promoted dtype.  Every
  // workspace is the layer's own (kept between calls), so nothing here waits for the device, and
  // with a caller's output nothing is allocated after the first call: a result that promotes
  // from bf16 to f32 part-way down the stack keeps its bf16 part in a layer-owned buffer.
  const Dtype final_dt = out_dtype(x.dtype());
  const Adapter* fused = adapters_[0].is_lokr() ? nullptr : &adapters_[0];
  const size_t rest = fused ? 1 : 0;  // first adapter applied one at a time
  const Array* first_out = out_arg;
  Array mid;
  if (out_arg && adapters_.size() > rest) {
    Dtype d1 = promote(promote(x.dtype(), q.scales.dtype()), q.bias ? q.bias->dtype() : x.dtype());
    if (fused) d1 = promote(d1, promote(x.dtype(), fused->a.dtype()));
    if (d1 != final_dt) {
      if (!mid_ || mid_->shape() != out_arg->shape() || mid_->dtype() != d1)
        mid_ = std::make_shared<Array>(Array::empty(out_arg->shape(), d1));
      mid = *mid_;
      first_out = &mid;
    }
  }
  Array y = q.forward_fused(x, fused, MLXQ_ACT_NONE, s, first_out);
  const int xdt = abi_dtype(x.dtype(), "AdaptableLinear::forward");
  const int64_t K = x.dim(-1), N = q.weight.dim(0), M = K > 0 ? x.size() / K : 0;
  for (size_t i = rest; i < adapters_.size(); ++i) {
    const Adapter& ad = adapters_[i];
    if (ad.is_lokr()) {
      if (ad.delta.ndim() != 2 || ad.delta.dim(0) != N || ad.delta.dim(1) != K)
        throw Error(MLXQ_EINVAL, "AdaptableLinear: a LoKr delta must be [out, in]");
      const Dtype odt = promote(y.dtype(), x.dtype());
      Array out = odt == y.dtype() ? y : (out_arg ? *out_arg : Array::empty(y.shape(), odt));
      Array& ws = grow_workspace(workspace_, mlxq_lokr_residual_workspace_size(xdt, M, N));
      check(mlxq_lokr_residual(x.data(), xdt, M, K, ad.delta.data(),
                               abi_dtype(ad.delta.dtype(), "AdaptableLinear::forward"), N, ad.scale,
                               y.data(), abi_dtype(y.dtype(), "AdaptableLinear::forward"), out.data(),
                               ws.data(), ws.nbytes(), s));
      y = out;
      continue;
    }
    if (ad.a.ndim() != 2 || ad.b.ndim() != 2 || ad.a.dim(0) != K || ad.b.dim(1) != N ||
        ad.a.dim(1) != ad.b.dim(0) || ad.a.dtype() != ad.b.dtype())
      throw Error(MLXQ_EINVAL, "AdaptableLinear: LoRA factors must be A [in, r] and B [r, out] of one dtype");
    const int64_t rank = ad.a.dim(1);
    const int ldt = abi_dtype(ad.a.dtype(), "AdaptableLinear::forward");
    const Dtype odt = promote(y.dtype(), promote(x.dtype(), ad.a.dtype()));
    Array out = odt == y.dtype() ? y : (out_arg ? *out_arg : Array::empty(y.shape(), odt));
    Array& ws = grow_workspace(workspace_, mlxq_lora_residual_workspace_size(xdt, ldt, M, N, rank));
    check(mlxq_lora_residual(x.data(), xdt, M, K, ad.a.data(), ad.b.data(), ldt, N, rank, ad.scale,
                             y.data(), abi_dtype(y.dtype(), "AdaptableLinear::forward"), out.data(),
                             ws.data(), ws.nbytes(), s));
    y = out;
  }
  return y;
}

TokenEmbedding TokenEmbedding::dense(Array weight) {
  TokenEmbedding e;
  e.dense_ = std::move(weight);
  return e;
}

TokenEmbedding TokenEmbedding::from_quantized_parts(Array wq, Array scales, Array biases,
                                                    int group_size, int bits) {
  TokenEmbedding e;
  e.packed_ = Packed{std::move(wq), std::move(scales), std::move(biases)};
  e.group_size_ = group_size;
  e.bits_ = bits;
  return e;
}

Array TokenEmbedding::forward(const Array& ids, hipStream_t s) const {
  if (!packed_)
    throw Error(MLXQ_EUNSUPPORTED, "TokenEmbedding: the dense table is not on the quantized path");
  if (ids.dtype() != Dtype::Int32) throw Error(MLXQ_EINVAL, "TokenEmbedding: ids must be int32");
  const Packed& p = *packed_;
  const int64_t vocab = p.wq.dim(0), hidden = p.wq.dim(1) * 32 / bits_;
  std::vector<int64_t> shape = ids.shape();
  shape.push_back(hidden);
  Array out = Array::empty(shape, Dtype::Float32);
  check(mlxq_embedding((const int32_t*)ids.data(), ids.size(), (const uint32_t*)p.wq.data(),
                       p.scales.data(), p.biases.data(), abi_dtype(p.scales.dtype(), "embedding"),
                       vocab, hidden, group_size_, bits_, out.data(), MLXQ_FLOAT32, s));
  return out;
}

void TokenEmbedding::quantize(int bits, bool cast_to_bf16, hipStream_t s) {
  if (packed_) return;
  const Array w = cast_to_bf16 ? as_dtype(*dense_, Dtype::Bfloat16, s) : *dense_;
  packed_ = mlxq::quantize(w, 64, bits, s);
  group_size_ = 64;
  bits_ = bits;
  dense_.reset();
}

// ---- quant.rs ---------------------------------------------------------------------------------

const Array& require(const Weights& w, const std::string& key) {
  auto it = w.find(key);
  if (it == w.end()) throw Error(MLXQ_EINVAL, "missing tensor " + key);
  return it->second;
}

AdaptableLinear lin(const Weights& w, const std::string& base, bool bias, int group_size) {
  std::optional<Array> b;
  if (bias) b = require(w, base + ".bias");
  auto sc = w.find(base + ".scales");
  if (sc != w.end()) {
    const Array& wq = require(w, base + ".weight");
    const int bits = packed_bits(wq, sc->second, group_size);
    return AdaptableLinear::from_quantized_parts(wq, sc->second, require(w, base + ".biases"), b,
                                                 group_size, bits);
  }
  return AdaptableLinear::dense(require(w, base + ".weight"), b);
}

TokenEmbedding embedding(const Weights& w, const std::string& base, int group_size) {
  auto sc = w.find(base + ".scales");
  if (sc != w.end()) {
    const Array& wq = require(w, base + ".weight");
    const int bits = packed_bits(wq, sc->second, group_size);
    return TokenEmbedding::from_quantized_parts(wq, sc->second, require(w, base + ".biases"),
                                                group_size, bits);
  }
  return TokenEmbedding::dense(require(w, base + ".weight"));
}

bool has_packed_experts(const Weights& w, const std::string& prefix, const std::string& name) {
  return w.count(prefix + ".experts." + name + "_proj.scales") > 0;
}

StackedExperts load_packed_experts(const Weights& w, const std::string& prefix, const std::string& name) {
  const std::string base = prefix + ".experts." + name + "_proj";
  StackedExperts st;
  st.weight = require(w, base + ".weight");
  st.scales = require(w, base + ".scales");
  st.biases = require(w, base + ".biases");
  st.bias = require(w, prefix + ".experts." + name + "_proj_bias");
  st.group_size = 64;
  if (st.weight.ndim() != 3 || st.scales.ndim() != 3)
    throw Error(MLXQ_EINVAL, "load_packed_experts: expected [E, out, ...] stacks under " + base);
  st.bits = packed_bits(st.weight.index0(0), st.scales.index0(0), st.group_size);
  return st;
}

Weights quantize_map(const Weights& map, int bits, int group_size,
                     const std::function<bool(const std::string&)>& is_target, hipStream_t s) {
  // Targets of one shape are packed together (quantize_batched: the same triples as one quantize
  // per weight, fewer launches).
  static const std::string suffix = ".weight";
  Weights out;
  std::map<std::vector<int64_t>, std::vector<std::string>> groups;  // shape -> target keys
  for (const auto& [k, v] : map) {
    const bool is_weight = k.size() > suffix.size() && k.compare(k.size() - suffix.size(), suffix.size(), suffix) == 0;
    const std::string base = is_weight ? k.substr(0, k.size() - suffix.size()) : std::string();
    const bool packable = is_weight && is_target(base) && v.ndim() == 2 &&
                          group_size > 0 && v.dim(1) % group_size == 0 && v.dim(1) >= group_size;
    if (packable) groups[v.shape()].push_back(k);
    else out[k] = v;
  }
  for (const auto& [shape, keys] : groups) {
    std::vector<Array> ws;
    for (const std::string& k : keys) ws.push_back(as_dtype(map.at(k), Dtype::Bfloat16, s));
    const std::vector<Packed> ps = quantize_batched(ws, group_size, bits, s);
    for (size_t i = 0; i < keys.size(); ++i) {
      const std::string base = keys[i].substr(0, keys[i].size() - suffix.size());
      out[base + ".weight"] = ps[i].wq;
      out[base + ".scales"] = ps[i].scales;
      out[base + ".biases"] = ps[i].biases;
    }
  }
  return out;
}

}  // namespace mlxq
