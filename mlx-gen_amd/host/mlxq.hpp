// mlxq.hpp — C++ host API of the MI355X quantized-linear path, layered on the C ABI of
// libmlxq_hip.so (include/mlxq.h).
//
// It mirrors the reference's Rust surface for this path with the same names, argument meanings
// and error behaviour, so a caller ports line for line:
//   mlx_rs::ops::{quantize, dequantize, quantized_matmul}  (src/quant.rs:140, src/nn.rs:55,
//                                                           src/adapters.rs:309-317)
//   quant::{packed_bits, lin, embedding, load_dir_map, save_map, quantize_map}
//                                                          (src/quant.rs:38-149)
//   nn::QuantizedLinear, adapters::{Adapter, AdaptableLinear} (src/adapters.rs:231-549)
//   nn::TokenEmbedding                                     (src/nn.rs:20-101)
//   convert::write_quantized_config                        (mlx-gen-flux/src/convert.rs:46-63)
// Errors are thrown as mlxq::Error (the reference returns Result<_, Error>); a status code and
// the library's message travel with it.  Arrays are ref-counted device buffers: copying an Array
// copies the handle, as cloning an mlx_rs::Array does (src/quant.rs:92-94).
#pragma once

#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace mlxq {

// The first two values are the C ABI's mlxq_dtype; the others are storage types the loaders carry.
enum class Dtype : int {
  Float32 = 0, Bfloat16 = 1, Uint32 = 2, Int32 = 3, Float16 = 4, Int64 = 5, Uint8 = 6, Int8 = 7,
  Float64 = 8, Bool = 9
};
size_t dtype_size(Dtype dt);
const char* dtype_name(Dtype dt);       // safetensors spelling: F32, BF16, U32, I32, ...
Dtype dtype_from_name(const std::string& name);  // throws on an unknown spelling

class Error : public std::runtime_error {
 public:
  Error(int status, const std::string& msg) : std::runtime_error(msg), status(status) {}
  int status;  // mlxq_status
};

// Device array: shared ownership of a HIP allocation (or a borrowed pointer), row-major.
class Array {
 public:
  Array() = default;
  static Array empty(std::vector<int64_t> shape, Dtype dt);
  static Array from_host(const void* data, std::vector<int64_t> shape, Dtype dt);
  // Wraps memory owned elsewhere (e.g. a framework tensor); the caller keeps it alive.
  static Array borrow(void* device_ptr, std::vector<int64_t> shape, Dtype dt);
  // Two arrays of one shape in one allocation, the second starting 256 bytes past the first's
  // end rounded up: quantize's scales and biases, which the large-M GEMM stages through one
  // buffer resource reaching both (separate allocations may lie more than 4 GiB apart).
  static std::pair<Array, Array> empty_pair(std::vector<int64_t> shape, Dtype dt);

  void to_host(void* dst) const;  // synchronous device-to-host copy of nbytes()
  Array reshape(std::vector<int64_t> shape) const;  // same buffer, new shape (same size)
  // Sub-array i along axis 0 (shape without that axis), sharing this buffer, as split + squeeze
  // along axis 0 do for the stacked expert packs (mlx-gen-lens/src/quant.rs:111-137).
  Array index0(int64_t i) const;

  bool valid() const { return ptr_ != nullptr || size() == 0; }
  void* data() const { return ptr_; }
  const std::vector<int64_t>& shape() const { return shape_; }
  int ndim() const { return (int)shape_.size(); }
  int64_t dim(int i) const { return shape_.at(i < 0 ? shape_.size() + i : i); }
  int64_t size() const;
  size_t nbytes() const { return (size_t)size() * dtype_size(dtype_); }
  Dtype dtype() const { return dtype_; }

 private:
  std::shared_ptr<void> buf_;
  void* ptr_ = nullptr;
  std::vector<int64_t> shape_;
  Dtype dtype_ = Dtype::Float32;
};

// ---- ops (mlx_rs::ops) ----------------------------------------------------------------------
struct Packed {
  Array wq, scales, biases;
};
// `as_dtype` between f32 and bf16 (round to nearest even); returns `a` itself when equal.
Array as_dtype(const Array& a, Dtype dt, hipStream_t s = nullptr);
Packed quantize(const Array& w, int group_size, int bits, hipStream_t s = nullptr);
// quantize over weights of one shape and dtype, several per launch (mlxq_quantize_batched): the
// same triples as one quantize per weight.
std::vector<Packed> quantize_batched(const std::vector<Array>& ws, int group_size, int bits,
                                     hipStream_t s = nullptr);
Array dequantize(const Array& wq, const Array& scales, const Array& biases, int group_size, int bits,
                 hipStream_t s = nullptr);
// x [..., K] -> [..., N]; only transpose = true exists in the reference and here.
Array quantized_matmul(const Array& x, const Array& wq, const Array& scales, const Array& biases,
                       bool transpose, int group_size, int bits, hipStream_t s = nullptr);
int packed_bits(const Array& wq, const Array& scales, int group_size);

// ---- layers ---------------------------------------------------------------------------------
// One adapter of AdaptableLinear's stack (enum Adapter, src/adapters.rs:231-270):
//   LoRA: residual = scale * (x.A).B with A [in, r], B [r, out] (alpha/rank folded in B,
//         src/adapters/loader.rs:568-599), the factors in their file dtype;
//   LoKr: residual = scale * x . delta^T with delta [out, in] the reconstructed kron delta
//         (reconstruct_lokr_delta, src/adapters.rs:26-128), cast to the activation dtype.
struct Adapter {
  Array a, b;  // LoRA factors
  float scale = 1.0f;
  Array delta;  // LoKr delta (kind == Kind::Lokr)
  enum class Kind { Lora, Lokr } kind = Kind::Lora;

  static Adapter lora(Array a, Array b, float scale) { return Adapter{std::move(a), std::move(b), scale}; }
  static Adapter lokr(Array delta, float scale) {
    Adapter r;
    r.delta = std::move(delta);
    r.scale = scale;
    r.kind = Kind::Lokr;
    return r;
  }
  bool is_lokr() const { return kind == Kind::Lokr; }
};

struct QuantizedLinear {
  Array weight, scales, biases;  // packed triple (weight in U32)
  std::optional<Array> bias;     // dense bias (its own dtype: an f32 bias promotes, as in MLX)
  int group_size = 64;
  int bits = 4;

  static QuantizedLinear try_from_linear(const Array& weight, std::optional<Array> bias,
                                         int group_size, int bits, hipStream_t s = nullptr);
  // y = x . W^T (+ bias), in MLX's promoted dtype.
  Array forward(const Array& x, hipStream_t s = nullptr) const;
  // forward with one LoRA adapter and an mlxq_activation fused after it (mlxq_linear); the
  // result goes to *out when given (shape and dtype checked), else to a new array.
  Array forward_fused(const Array& x, const Adapter* lora, int activation, hipStream_t s = nullptr,
                      const Array* out = nullptr) const;
  int64_t in_features() const { return scales.dim(1) * group_size; }

  // Device workspace of mlxq_linear, kept with the layer and grown on demand, so that forward
  // calls after the first allocate none (last member: aggregate initialisation leaves it empty).
  // Calls on one layer must be ordered on one stream.
  mutable std::shared_ptr<Array> workspace_;
};

class AdaptableLinear {
 public:
  static AdaptableLinear dense(Array weight, std::optional<Array> bias);
  static AdaptableLinear from_quantized_parts(Array weight, Array scales, Array biases,
                                              std::optional<Array> bias, int group_size, int bits);
  void push(Adapter a) { adapters_.push_back(std::move(a)); }
  void set_adapters(std::vector<Adapter> a) { adapters_ = std::move(a); }
  const std::vector<Adapter>& adapters() const { return adapters_; }
  bool is_quantized() const { return quantized_.has_value(); }
  const QuantizedLinear& quantized() const { return quantized_.value(); }
  std::array<int64_t, 2> base_shape() const;
  // src/adapters.rs:508-541: cast weight and bias to bf16, then pack; no-op when packed.
  void quantize(int bits, std::optional<int> group_size, hipStream_t s = nullptr);
  // src/adapters.rs:300-322,543-549: base(x) (+ bias) + sum of adapter residuals, each step
  // rounded to its promoted dtype (bias and factors keep their own dtypes, as in MLX).  The dense
  // base is not on this library's path and throws.  Workspaces are the layer's own and kept
  // between calls: calls on one layer must be ordered on one stream.
  Array forward(const Array& x, hipStream_t s = nullptr) const;
  // forward into a caller's array of shape [..., out] and dtype out_dtype(x.dtype()): after a
  // first call with the same shapes this allocates nothing and never waits for the device, so it
  // can be captured into a HIP graph.
  void forward_into(const Array& x, const Array& out, hipStream_t s = nullptr) const;
  Dtype out_dtype(Dtype x_dtype) const;

 private:
  Array forward_impl(const Array& x, const Array* out, hipStream_t s) const;
  std::optional<Array> dense_weight_, dense_bias_;
  std::optional<QuantizedLinear> quantized_;
  std::vector<Adapter> adapters_;
  mutable std::shared_ptr<Array> workspace_;  // mlxq_{lora,lokr}_residual staging, grown on demand
  mutable std::shared_ptr<Array> mid_;        // a bf16 partial sum before an f32 adapter
};

class TokenEmbedding {
 public:
  static TokenEmbedding dense(Array weight);
  static TokenEmbedding from_quantized_parts(Array wq, Array scales, Array biases, int group_size,
                                             int bits);
  bool is_quantized() const { return packed_.has_value(); }
  int group_size() const { return group_size_; }
  int bits() const { return bits_; }
  const Packed& packed() const { return packed_.value(); }
  // ids (int32, any shape) -> [..., hidden] f32.  Only the packed table runs here.
  Array forward(const Array& ids, hipStream_t s = nullptr) const;
  // Pack with group size 64 (bf16 first when cast_to_bf16); no-op when packed.
  void quantize(int bits, bool cast_to_bf16, hipStream_t s = nullptr);

 private:
  std::optional<Array> dense_;
  std::optional<Packed> packed_;
  int group_size_ = 64, bits_ = 4;
};

// Fused SwiGLU of a decode MLP (mlx-gen-sensenova/src/qwen3.rs:178-181): h = silu(gate(x)) * up(x)
// with both projections streamed in one launch.  Decode form only (bf16 x and scales, M <= 8,
// no dense bias); other inputs throw Error(MLXQ_EUNSUPPORTED) and the caller runs two forwards.
Array swiglu(const Array& x, const QuantizedLinear& gate, const QuantizedLinear& up,
             hipStream_t s = nullptr);

// One MoE expert projection across all E experts as its stacked packed triple plus dense bias
// (mlx-gen-lens/src/text_encoder/gpt_oss.rs:478-487): weight [E, out, in*bits/32], scales/biases
// [E, out, in/group_size], bias [E, out].
struct StackedExperts {
  Array weight, scales, biases;
  std::optional<Array> bias;
  int group_size = 64;
  int bits = 4;

  int64_t num_experts() const { return weight.dim(0); }
  // Per-expert layers sharing the stack's buffers (the axis-0 split of quant.rs:111-137); an
  // expert's scales/biases slice that starts mid-word is copied instead.
  std::vector<QuantizedLinear> split() const;
  // Proj::forward of every expert (gpt_oss.rs:412-425) in one call: x [..., in] shared by all
  // experts, or [E, ..., in] with per_expert; returns [E, ..., out].
  Array forward(const Array& x, bool per_expert = false, hipStream_t s = nullptr) const;
};

// ---- quant.rs --------------------------------------------------------------------------------
using Weights = std::map<std::string, Array>;
const Array& require(const Weights& w, const std::string& key);  // throws on a missing key
AdaptableLinear lin(const Weights& w, const std::string& base, bool bias, int group_size);
TokenEmbedding embedding(const Weights& w, const std::string& base, int group_size);
// mlx-gen-lens/src/quant.rs:80-137: `{prefix}.experts.{name}_proj.{weight,scales,biases}` stacks
// plus `{prefix}.experts.{name}_proj_bias`; bits from the packed shapes, group size 64.
bool has_packed_experts(const Weights& w, const std::string& prefix, const std::string& name);
StackedExperts load_packed_experts(const Weights& w, const std::string& prefix, const std::string& name);
Weights quantize_map(const Weights& map, int bits, int group_size,
                     const std::function<bool(const std::string&)>& is_target,
                     hipStream_t s = nullptr);

// ---- snapshot I/O ----------------------------------------------------------------------------
struct HostTensor {
  Dtype dtype = Dtype::Float32;
  std::vector<int64_t> shape;
  std::vector<uint8_t> data;
};
using HostMap = std::map<std::string, HostTensor>;
HostMap read_safetensors(const std::string& path);
void write_safetensors(const std::string& path, const HostMap& tensors);
Weights load_dir_map(const std::string& dir);                 // every *.safetensors in dir
void save_map(const std::string& path, const Weights& map);   // one file
void write_quantized_config(const std::string& src_dir, const std::string& dst_dir, int bits,
                            int group_size);

}  // namespace mlxq
