// compute.hpp — the C++ host side of the ROCm backend: fak's compute HAL seam restated over the
// fakhip C ABI (include/fakhip.h).
//
// The Go engine selects a device through compute.Backend (internal/compute/compute.go:318-347)
// and a registry (Register / Registered / Lookup / Pick / Default / RequireReference,
// compute.go:464-525). Its CUDA tenant (internal/compute/cuda.go) implements Upload / Read /
// Free / MatMul / BatchedMatMul over a flat C ABI. This header gives the same types and
// methods, with the same names, argument meaning and failure behaviour, for a C++ host of the
// gfx950 backend: a Go panic is a C++ exception (std::invalid_argument for a bad argument,
// std::runtime_error for a device failure, carrying fhip_last_error()).
//
// Only the quantized weight path is implemented: RMSNorm / RoPE / SwiGLU / attention and the
// f32 GEMMs belong to other kernels and throw std::logic_error.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace fak {
namespace compute {

// internal/compute/compute.go:53-64 (same order and values).
enum class Dtype : int { F32 = 0, F16 = 1, BF16 = 2, Q8_0 = 3, I8 = 4, I4 = 5, FP8 = 6, Q4_K = 7 };
std::string to_string(Dtype d);  // compute.go:80-101 ("f32", "q4_k", ...)

// compute.go:113-117.
enum class Layout : int { RowMajor = 0, ColMajor = 1, Tiled = 2 };

// compute.go:212-217.
enum class CorrectnessClass : int { Reference = 0, Approx = 1 };
std::string to_string(CorrectnessClass c);

// compute.go:130-141.
struct QuantSpec {
  int Block = 0;
  int Axis = 0;
  int Bits = 0;
  bool Symmetric = false;
  std::vector<float> Scale;  // per-block scales of a host Q8_0 weight
};

// compute.go:234-256 (the fields this backend sets).
struct Caps {
  bool Async = false;
  bool FusedAttn = false;
  bool FusedFFN = false;
  bool GraphCompile = false;
  bool UploadDtype = false;
  bool DeviceMemory = false;
  bool Collective = false;
  bool CapacityProbe = false;
};

struct Buffer {
  virtual ~Buffer() = default;
  virtual bool Ready() const { return true; }
};

// The reference's hostBuf: an f32 view or an int8 view of host data. gguf_blocks marks raw GGUF
// Q8_0 blocks (f16 d + 32 int8) rather than HAL int8 codes.
struct HostBuffer : Buffer {
  std::vector<float> f32;
  std::vector<int8_t> i8;
  bool gguf_blocks = false;
};

// A device allocation from the fakhip pool. HAL Q8 weights carry a second (scales) buffer.
// An async op output (a matmul result) records the fence generation it was enqueued in and is
// Ready() only once a host fence (Read) has bumped its backend's generation past it
// (cudaBuf.Ready, internal/compute/cuda.go:286-300): the stream is FIFO, so one fence
// materializes every buffer enqueued before it. Buffers with no fence counter (uploads, which
// complete before they return) are always ready.
struct DeviceBuffer : Buffer {
  void *ptr = nullptr;
  size_t bytes = 0;
  void *scales = nullptr;
  int block = 0;
  std::shared_ptr<const std::atomic<uint64_t>> fence;
  uint64_t born_gen = 0;
  bool Ready() const override { return !fence || fence->load() > born_gen; }
};

class Backend;

// compute.go:168-175.
struct Tensor {
  Dtype dtype = Dtype::F32;
  Layout layout = Layout::RowMajor;
  std::vector<int> shape;
  std::shared_ptr<QuantSpec> quant;
  std::shared_ptr<Buffer> buf;
  Backend *be = nullptr;

  long long Numel() const;
  const HostBuffer *host() const { return dynamic_cast<const HostBuffer *>(buf.get()); }
  DeviceBuffer *device() const { return dynamic_cast<DeviceBuffer *>(buf.get()); }
};

// Host tensor constructors: NewF32 (internal/compute/cpuref.go:47-49), NewQ4K (raw GGUF Q4_K
// bytes, internal/compute/quant_q4k.go:37-44), NewQ8 (int8 codes + f32 block scales,
// cpuref.go:53-56) and NewQ8_0GGUF (raw GGUF Q8_0 blocks; the scale of each block recorded as
// its exact f32 widening, the values of the reference's resident kqw Q8_0 weight).
Tensor NewF32(Backend *be, std::vector<int> shape, std::vector<float> data);
Tensor NewQ4K(Backend *be, std::vector<int> shape, const std::vector<uint8_t> &raw);
Tensor NewQ8(Backend *be, std::vector<int> shape, std::vector<int8_t> codes,
             std::vector<float> scale, int block = 32);
Tensor NewQ8_0GGUF(Backend *be, std::vector<int> shape, const std::vector<uint8_t> &raw);

class Backend {
 public:
  virtual ~Backend() = default;
  virtual std::string Name() const = 0;
  virtual std::string Tier() const = 0;
  virtual CorrectnessClass Class() const = 0;
  virtual compute::Caps Caps() const = 0;

  virtual Tensor Upload(const Tensor &t, Dtype as) = 0;
  // Host-addressable f32 view, or false on a device backend.
  virtual bool Host(const Tensor &t, std::vector<float> *out) {
    (void)t;
    (void)out;
    return false;
  }
  virtual std::vector<float> Read(const Tensor &t) = 0;
  virtual void Free(Tensor &t) = 0;

  virtual Tensor MatMul(const Tensor &w, const Tensor &x) = 0;
  virtual Tensor BatchedMatMul(const Tensor &w, const Tensor &X, int P) = 0;

  // The rest of the interface (compute.go:331-346) belongs to other kernels.
  virtual Tensor RMSNorm(const Tensor &, const Tensor &, float) { return unsupported("RMSNorm"); }
  virtual Tensor RoPE(const Tensor &, int, int, int, double) { return unsupported("RoPE"); }
  virtual Tensor SwiGLU(const Tensor &, const Tensor &) { return unsupported("SwiGLU"); }
  virtual void AddInPlace(Tensor &, const Tensor &) { unsupported("AddInPlace"); }
  virtual void AddBias(Tensor &, const Tensor &) { unsupported("AddBias"); }
  virtual int Argmax(const Tensor &) {
    unsupported("Argmax");
    return -1;
  }

 protected:
  Tensor unsupported(const char *op) const;
};

// The gfx950 Approx backend over the fakhip C ABI: the restatement of cudaBackend
// (internal/compute/cuda.go:212-232 registration, 690-750 and 803-836 upload, 956-1035 matmul).
class RocmBackend : public Backend {
 public:
  // Initialises device 0 (fhip_init); throws std::runtime_error without a gfx950 device.
  // kq_int8 < 0 reads FAK_KQ_INT8 (1 / on / true) like q4kInt8Default
  // (internal/model/quant_amd64_q4k.go:54-61); 0 / 1 force the route.
  explicit RocmBackend(int kq_int8 = -1);
  ~RocmBackend() override;

  std::string Name() const override { return "rocm"; }
  std::string Tier() const override { return tier_; }
  CorrectnessClass Class() const override { return CorrectnessClass::Approx; }
  compute::Caps Caps() const override;

  Tensor Upload(const Tensor &t, Dtype as) override;
  std::vector<float> Read(const Tensor &t) override;
  void Free(Tensor &t) override;
  Tensor MatMul(const Tensor &w, const Tensor &x) override;
  Tensor BatchedMatMul(const Tensor &w, const Tensor &X, int P) override;

  bool kq_int8() const { return kq_int8_; }
  // Device bytes a resident weight occupies (codes + scales for HAL Q8; the tiled records for
  // Q4_K / Q8_0 blocks), read off its device buffers.
  static size_t ResidentBytes(const Tensor &w);

 private:
  Tensor upload_quant(const Tensor &t, int block, int block_bytes);
  Tensor upload_hal_q8(const Tensor &t);
  Tensor narrow_q8(const Tensor &t);
  Tensor matmul(const Tensor &w, const Tensor &X, int P, std::vector<int> shape);
  Tensor dev_out(std::vector<int> shape);
  // The resident copy of host tensor `t` made earlier (same host buffer object, still alive,
  // same dtype and element count: cuda.go:690-704), or an empty tensor.
  Tensor cached(const Tensor &t, Dtype d) const;
  void remember(const Tensor &host, Dtype d, const Tensor &resident);

  struct CacheEntry {
    std::weak_ptr<Buffer> host;  // expired once the host tensor is gone: never a stale hit
    Dtype dtype;
    Tensor t;
  };
  // Host fences (Read) so far (cudaBackend.fenceGen, cuda.go:327-331); shared with the async
  // outputs so their Ready() stays valid after the backend is gone.
  std::shared_ptr<std::atomic<uint64_t>> fence_gen_ = std::make_shared<std::atomic<uint64_t>>(0);
  std::vector<CacheEntry> cache_;
  std::string tier_;
  bool kq_int8_ = false;
};

// ---- registry (compute.go:464-525) ----
void Register(std::shared_ptr<Backend> b);
std::vector<std::string> Registered();
std::shared_ptr<Backend> Lookup(const std::string &name, bool *ok);
std::shared_ptr<Backend> Pick(const std::string &name);
std::shared_ptr<Backend> Default();
bool RequireReference(const Backend *b);
// The init() of cuda.go:212-232: register "rocm" when a gfx950 device is reachable; returns
// whether it registered (no device: registers nothing).
bool RegisterRocm();
// Empties the registry (tests).
void ResetRegistry();

// ---- model-level seams (no compute.Dtype in the reference) ----

// A resident Q6_K weight [Out, In] (the q4_k_m ffn_down / output quant): the device twin of
// metalgemm.Q6KWeight / UploadQ6K (internal/metalgemm/q4k.go:163-190). Empty (ptr null) when
// the shape is bad or the payload short, as UploadQ6K returns nil.
struct Q6KWeight {
  void *ptr = nullptr;
  int Out = 0, In = 0;
  explicit operator bool() const { return ptr != nullptr; }
};
Q6KWeight UploadQ6K(const uint8_t *raw, size_t len, int out, int in);
void FreeQ6K(Q6KWeight &w);
// y[P][Out] = X[P][In] @ W^T on device buffers (kQuantMatRowsInto(kind Q6_K)).
void Q6KMatRows(const Q6KWeight &w, const Tensor &X, Tensor &Y, int P);

// The fused dense SwiGLU MLP of a decode step, y = down(silu(gate x) * (up x)), over resident
// Q4_K gate / up / down (FusedMLP, internal/metalgemm/q4k.go:144-161) or a Q6_K down
// (FusedMLPQ6Down, :192-205). x and y are device F32 tensors of [P, H]. Returns false on a shape
// mismatch (the caller then runs the per-matmul path), as the reference does.
bool FusedMLP(const Tensor &gate, const Tensor &up, const Tensor &down, const Tensor &x,
              Tensor &y, int P = 1);
bool FusedMLPQ6Down(const Tensor &gate, const Tensor &up, const Q6KWeight &down,
                    const Tensor &x, Tensor &y, int P = 1);

}  // namespace compute
}  // namespace fak
