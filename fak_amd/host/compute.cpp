// compute.cpp — fak's compute HAL seam over the fakhip C ABI (see compute.hpp).
#include "compute.hpp"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "fakhip.h"

namespace fak {
namespace compute {

namespace {

[[noreturn]] void device_fail(const char *fn, int rc) {
  throw std::runtime_error(std::string(fn) + " failed with status " + std::to_string(rc) + ": " +
                           fhip_last_error());
}

void check(const char *fn, int rc) {
  if (rc != FHIP_OK) device_fail(fn, rc);
}

void *alloc(size_t bytes) {
  void *p = fhip_malloc(bytes ? bytes : 4);
  if (!p) device_fail("fhip_malloc", FHIP_ENOMEM);
  return p;
}

std::string shape_str(const std::vector<int> &s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
  return o + "]";
}

// IEEE half -> single, subnormals included (the exact widening of a stored f16 scale).
float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int exp = (h >> 10) & 0x1f;
  uint32_t frac = h & 0x3ffu, bits;
  if (exp == 0) {
    if (frac == 0) {
      bits = sign;
    } else {
      exp = -14;
      while (!(frac & 0x400u)) {
        frac <<= 1;
        --exp;
      }
      bits = sign | (uint32_t)(exp + 127) << 23 | (frac & 0x3ffu) << 13;
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | frac << 13;
  } else {
    bits = sign | (uint32_t)(exp - 15 + 127) << 23 | frac << 13;
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

std::mutex g_reg_mu;
std::vector<std::shared_ptr<Backend>> g_registry;

// q8DeviceBlock, internal/compute/cuda.go:210.
constexpr int kQ8DeviceBlock = 32;

}  // namespace

std::string to_string(Dtype d) {
  switch (d) {
    case Dtype::F32: return "f32";
    case Dtype::F16: return "f16";
    case Dtype::BF16: return "bf16";
    case Dtype::Q8_0: return "q8_0";
    case Dtype::I8: return "i8";
    case Dtype::I4: return "i4";
    case Dtype::FP8: return "fp8";
    case Dtype::Q4_K: return "q4_k";
  }
  return "dtype?";
}

std::string to_string(CorrectnessClass c) {
  return c == CorrectnessClass::Reference ? "reference" : "approx";
}

long long Tensor::Numel() const {
  long long n = 1;
  for (int d : shape) n *= d;
  return n;
}

Tensor Backend::unsupported(const char *op) const {
  throw std::logic_error("compute: " + Name() + " backend implements the quantized matmul only (" +
                         op + ")");
}

// ---- host tensors ----

Tensor NewF32(Backend *be, std::vector<int> shape, std::vector<float> data) {
  Tensor t;
  t.dtype = Dtype::F32;
  t.shape = std::move(shape);
  auto hb = std::make_shared<HostBuffer>();
  hb->f32 = std::move(data);
  t.buf = hb;
  t.be = be;
  return t;
}

Tensor NewQ4K(Backend *be, std::vector<int> shape, const std::vector<uint8_t> &raw) {
  Tensor t;
  t.dtype = Dtype::Q4_K;
  t.shape = std::move(shape);
  t.quant = std::make_shared<QuantSpec>();
  t.quant->Block = 256;
  t.quant->Axis = 2;
  t.quant->Bits = 4;
  t.quant->Symmetric = false;
  auto hb = std::make_shared<HostBuffer>();
  hb->i8.assign(reinterpret_cast<const int8_t *>(raw.data()),
                reinterpret_cast<const int8_t *>(raw.data()) + raw.size());
  t.buf = hb;
  t.be = be;
  return t;
}

Tensor NewQ8(Backend *be, std::vector<int> shape, std::vector<int8_t> codes,
             std::vector<float> scale, int block) {
  Tensor t;
  t.dtype = Dtype::Q8_0;
  t.shape = std::move(shape);
  t.quant = std::make_shared<QuantSpec>();
  t.quant->Block = block;
  t.quant->Axis = 2;
  t.quant->Bits = 8;
  t.quant->Symmetric = true;
  t.quant->Scale = std::move(scale);
  auto hb = std::make_shared<HostBuffer>();
  hb->i8 = std::move(codes);
  t.buf = hb;
  t.be = be;
  return t;
}

Tensor NewQ8_0GGUF(Backend *be, std::vector<int> shape, const std::vector<uint8_t> &raw) {
  if (shape.size() != 2 || shape[1] % 32 ||
      raw.size() != (size_t)shape[0] * (shape[1] / 32) * 34)
    throw std::invalid_argument("compute: NewQ8_0GGUF " + shape_str(shape) + " with " +
                                std::to_string(raw.size()) + " bytes");
  const size_t nb = raw.size() / 34;
  std::vector<float> scale(nb);
  for (size_t b = 0; b < nb; ++b)
    scale[b] = half_to_float((uint16_t)(raw[34 * b] | raw[34 * b + 1] << 8));
  Tensor t;
  t.dtype = Dtype::Q8_0;
  t.shape = std::move(shape);
  t.quant = std::make_shared<QuantSpec>();
  t.quant->Block = 32;
  t.quant->Axis = 2;
  t.quant->Bits = 8;
  t.quant->Symmetric = true;
  t.quant->Scale = std::move(scale);
  auto hb = std::make_shared<HostBuffer>();
  hb->i8.assign(reinterpret_cast<const int8_t *>(raw.data()),
                reinterpret_cast<const int8_t *>(raw.data()) + raw.size());
  hb->gguf_blocks = true;
  t.buf = hb;
  t.be = be;
  return t;
}

// ---- RocmBackend ----

RocmBackend::RocmBackend(int kq_int8) {
  char name[256];
  int arch = 0;
  size_t total = 0;
  check("fhip_init", fhip_init(name, sizeof name, &arch, &total));
  tier_ = "gfx" + std::to_string(arch);
  if (kq_int8 < 0) {
    const char *v = std::getenv("FAK_KQ_INT8");
    const std::string s = v ? v : "";
    kq_int8_ = s == "1" || s == "on" || s == "true";
  } else {
    kq_int8_ = kq_int8 != 0;
  }
}

RocmBackend::~RocmBackend() = default;

compute::Caps RocmBackend::Caps() const {
  compute::Caps c;
  c.Async = true;
  c.UploadDtype = true;
  c.DeviceMemory = true;
  c.CapacityProbe = true;
  return c;
}

Tensor RocmBackend::cached(const Tensor &t, Dtype d) const {
  for (const auto &e : cache_) {
    auto h = e.host.lock();
    if (h && h == t.buf && e.dtype == d && e.t.Numel() == t.Numel()) return e.t;
  }
  return Tensor{};
}

void RocmBackend::remember(const Tensor &host, Dtype d, const Tensor &resident) {
  cache_.erase(std::remove_if(cache_.begin(), cache_.end(),
                              [](const CacheEntry &e) { return e.host.expired(); }),
               cache_.end());
  cache_.push_back({host.buf, d, resident});
}

Tensor RocmBackend::Upload(const Tensor &t, Dtype as) {
  const HostBuffer *hb = t.host();
  if (!hb) throw std::invalid_argument("compute: rocm Upload expects host data");
  if (t.dtype == Dtype::Q4_K) return upload_quant(t, 256, 144);
  if (t.dtype == Dtype::Q8_0 && hb->gguf_blocks) return upload_quant(t, 32, 34);
  if (t.dtype == Dtype::Q8_0) return upload_hal_q8(t);
  if (t.dtype != Dtype::F32)
    throw std::invalid_argument("compute: rocm Upload supports F32 host data, raw Q4_K / Q8_0 "
                                "blocks or HAL Q8 codes (got " + to_string(t.dtype) + ")");
  if (as == Dtype::Q8_0) return narrow_q8(t);
  const size_t n = hb->f32.size() * 4;
  auto db = std::make_shared<DeviceBuffer>();
  db->ptr = alloc(n);
  db->bytes = n;
  if (n) check("fhip_h2d", fhip_h2d(db->ptr, hb->f32.data(), n));
  Tensor r;
  r.dtype = Dtype::F32;
  r.shape = t.shape;
  r.buf = db;
  r.be = this;
  return r;
}

Tensor RocmBackend::upload_quant(const Tensor &t, int block, int block_bytes) {
  if (t.shape.size() != 2)
    throw std::invalid_argument("compute: rocm Upload(" + to_string(t.dtype) +
                                ") expects a 2-D [out,in] weight");
  const int out = t.shape[0], in = t.shape[1];
  const auto &raw = t.host()->i8;
  if (out <= 0 || in <= 0 || in % block)
    throw std::invalid_argument("compute: " + to_string(t.dtype) + " reduction dim " +
                                std::to_string(in) + " not a multiple of " + std::to_string(block));
  const size_t want = (size_t)out * (in / block) * block_bytes;
  if (raw.size() != want)
    throw std::invalid_argument("compute: " + to_string(t.dtype) + " payload size " +
                                std::to_string(raw.size()) + " != " + std::to_string(want));
  Tensor hit = cached(t, t.dtype);
  if (hit.buf) return hit;
  const uint8_t *src = reinterpret_cast<const uint8_t *>(raw.data());
  void *p = t.dtype == Dtype::Q4_K ? fhip_q4k_upload(src, out, in) : fhip_q8_0_upload(src, out, in);
  if (!p) device_fail(t.dtype == Dtype::Q4_K ? "fhip_q4k_upload" : "fhip_q8_0_upload", FHIP_ENOMEM);
  auto db = std::make_shared<DeviceBuffer>();
  db->ptr = p;
  db->bytes = t.dtype == Dtype::Q4_K ? fhip_q4k_packed_bytes(out, in)
                                     : fhip_q8_0_packed_bytes(out, in);
  Tensor r;
  r.dtype = t.dtype;
  r.layout = Layout::Tiled;
  r.shape = t.shape;
  r.quant = t.quant;
  r.buf = db;
  r.be = this;
  remember(t, t.dtype, r);
  return r;
}

Tensor RocmBackend::upload_hal_q8(const Tensor &t) {
  if (t.shape.size() != 2 || !t.quant)
    throw std::invalid_argument("compute: rocm Upload(Q8_0) expects a 2-D NewQ8 weight");
  const int out = t.shape[0], in = t.shape[1], block = t.quant->Block;
  const auto &codes = t.host()->i8;
  const auto &scale = t.quant->Scale;
  if (block <= 0 || in % block || codes.size() != (size_t)out * in ||
      scale.size() != (size_t)out * (in / block))
    throw std::invalid_argument("compute: Q8_0 weight " + shape_str(t.shape) + " block " +
                                std::to_string(block) + " has " + std::to_string(codes.size()) +
                                " codes / " + std::to_string(scale.size()) + " scales");
  Tensor hit = cached(t, Dtype::Q8_0);
  if (hit.buf) return hit;
  auto db = std::make_shared<DeviceBuffer>();
  db->ptr = alloc(codes.size());
  db->scales = alloc(scale.size() * 4);
  db->bytes = codes.size() + scale.size() * 4;
  db->block = block;
  if (!codes.empty()) {
    check("fhip_h2d", fhip_h2d(db->ptr, codes.data(), codes.size()));
    check("fhip_h2d", fhip_h2d(db->scales, scale.data(), scale.size() * 4));
  }
  Tensor r;
  r.dtype = Dtype::Q8_0;
  r.shape = t.shape;
  r.quant = t.quant;
  r.buf = db;
  r.be = this;
  remember(t, Dtype::Q8_0, r);
  return r;
}

// Upload(f32 weight, Q8_0): quantizeVecQ8 per row with the device block (cuda.go:714-750), run on
// the device.
Tensor RocmBackend::narrow_q8(const Tensor &t) {
  if (t.shape.size() != 2)
    throw std::invalid_argument("compute: rocm Upload(_, Q8_0) expects a 2-D [out,in] weight");
  const int out = t.shape[0], in = t.shape[1], blk = kQ8DeviceBlock;
  if (in % blk)
    throw std::invalid_argument("compute: Q8_0 reduction dim " + std::to_string(in) +
                                " not a multiple of " + std::to_string(blk));
  const auto &f = t.host()->f32;
  if (f.size() != (size_t)out * in)
    throw std::invalid_argument("compute: f32 weight has " + std::to_string(f.size()) +
                                " elements, want " + shape_str(t.shape));
  Tensor hit = cached(t, Dtype::Q8_0);
  if (hit.buf) return hit;
  const int nblk = in / blk;
  auto db = std::make_shared<DeviceBuffer>();
  db->ptr = alloc((size_t)out * in);
  db->scales = alloc((size_t)out * nblk * 4);
  db->bytes = (size_t)out * in + (size_t)out * nblk * 4;
  db->block = blk;
  if (!f.empty()) {
    void *tmp = alloc(f.size() * 4);
    int rc = fhip_h2d(tmp, f.data(), f.size() * 4);
    if (rc == FHIP_OK)
      rc = fhip_q8_quantize_f32((const float *)tmp, (int8_t *)db->ptr, (float *)db->scales, out,
                                in, blk);
    if (rc == FHIP_OK) rc = fhip_sync();
    fhip_free(tmp);
    check("fhip_q8_quantize_f32", rc);
  }
  Tensor r;
  r.dtype = Dtype::Q8_0;
  r.shape = t.shape;
  r.quant = std::make_shared<QuantSpec>();
  r.quant->Block = blk;
  r.quant->Axis = 2;
  r.quant->Bits = 8;
  r.quant->Symmetric = true;
  r.buf = db;
  r.be = this;
  remember(t, Dtype::Q8_0, r);
  return r;
}

std::vector<float> RocmBackend::Read(const Tensor &t) {
  if (t.dtype != Dtype::F32) throw std::invalid_argument("compute: rocm Read supports F32 tensors");
  const DeviceBuffer *db = t.device();
  if (!db || !db->ptr) throw std::invalid_argument("compute: rocm Read of a non-resident tensor");
  std::vector<float> out((size_t)t.Numel());
  if (!out.empty()) {
    check("fhip_d2h", fhip_d2h(out.data(), db->ptr, out.size() * 4));
    // The copy drained the stream: everything enqueued before it is materialized (cuda.go:896).
    fence_gen_->fetch_add(1);
  }
  return out;
}

void RocmBackend::Free(Tensor &t) {
  DeviceBuffer *db = t.device();
  if (!db || !db->ptr) return;
  cache_.erase(std::remove_if(cache_.begin(), cache_.end(),
                              [&](const CacheEntry &e) { return e.t.buf.get() == db; }),
               cache_.end());
  fhip_free(db->ptr);
  db->ptr = nullptr;
  if (db->scales) {
    fhip_free(db->scales);
    db->scales = nullptr;
  }
}

size_t RocmBackend::ResidentBytes(const Tensor &w) {
  const DeviceBuffer *db = w.device();
  return db && db->ptr ? db->bytes : 0;
}

Tensor RocmBackend::dev_out(std::vector<int> shape) {
  Tensor r;
  r.dtype = Dtype::F32;
  r.shape = std::move(shape);
  auto db = std::make_shared<DeviceBuffer>();
  db->bytes = (size_t)r.Numel() * 4;
  db->ptr = alloc(db->bytes);
  // An async output: not Ready() until the next host fence (cuda.go:583-596).
  db->fence = fence_gen_;
  db->born_gen = fence_gen_->load();
  r.buf = db;
  r.be = this;
  return r;
}

Tensor RocmBackend::matmul(const Tensor &w, const Tensor &X, int P, std::vector<int> shape) {
  const DeviceBuffer *wb = w.device();
  if (w.shape.size() != 2 || !wb || !wb->ptr)
    throw std::invalid_argument("compute: rocm MatMul expects a resident 2-D weight");
  const int out = w.shape[0], in = w.shape[1];
  const DeviceBuffer *xb = X.device();
  if (X.dtype != Dtype::F32 || !xb || !xb->ptr)
    throw std::invalid_argument("compute: rocm MatMul expects a device-resident F32 activation");
  if (P < 0 || X.Numel() != (long long)P * in)
    throw std::invalid_argument("compute: rocm MatMul activation has " +
                                std::to_string(X.Numel()) + " elements, want " +
                                std::to_string(P) + "x" + std::to_string(in));
  Tensor y = dev_out(std::move(shape));
  float *dy = (float *)y.device()->ptr;
  const float *dx = (const float *)xb->ptr;
  if (w.dtype == Dtype::Q4_K) {
    if (kq_int8_)
      check("fhip_q4k_matmul_int8_f32", fhip_q4k_matmul_int8_f32(wb->ptr, dx, dy, out, in, P));
    else
      check("fhip_q4k_matmul_f32", fhip_q4k_matmul_f32(wb->ptr, dx, dy, out, in, P));
  } else if (w.dtype == Dtype::Q8_0 && wb->scales) {
    check("fhip_q8_matmul_f32", fhip_q8_matmul_f32((const int8_t *)wb->ptr,
                                                   (const float *)wb->scales, dx, dy, out, in,
                                                   P, wb->block));
  } else if (w.dtype == Dtype::Q8_0) {
    check("fhip_q8_0_matmul_f32", fhip_q8_0_matmul_f32(wb->ptr, dx, dy, out, in, P));
  } else {
    throw std::logic_error("compute: rocm MatMul supports Q4_K / Q8_0 weights (got " +
                           to_string(w.dtype) + ")");
  }
  return y;
}

Tensor RocmBackend::MatMul(const Tensor &w, const Tensor &x) {
  if (w.shape.size() != 2) throw std::invalid_argument("compute: rocm MatMul expects [out,in]");
  const int out = w.shape[0];
  Tensor y = matmul(w, x, 1, {out});
  if (y.Numel() != out)  // cuda.go:989-993
    throw std::runtime_error("compute: rocm MatMul " + to_string(w.dtype) + " out=" +
                             std::to_string(out) + " produced " + std::to_string(y.Numel()) +
                             " rows");
  return y;
}

Tensor RocmBackend::BatchedMatMul(const Tensor &w, const Tensor &X, int P) {
  if (w.shape.size() != 2) throw std::invalid_argument("compute: rocm MatMul expects [out,in]");
  const int out = w.shape[0];
  Tensor y = matmul(w, X, P, {P, out});
  if (y.Numel() != (long long)P * out)  // cuda.go:1029-1033
    throw std::runtime_error("compute: rocm BatchedMatMul " + to_string(w.dtype) + " P=" +
                             std::to_string(P) + " produced " + std::to_string(y.Numel()));
  return y;
}

// ---- registry ----

void Register(std::shared_ptr<Backend> b) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  for (auto &e : g_registry)
    if (e->Name() == b->Name()) {
      e = std::move(b);
      return;
    }
  g_registry.push_back(std::move(b));
}

std::vector<std::string> Registered() {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  std::vector<std::string> out;
  for (auto &b : g_registry) out.push_back(b->Name());
  return out;
}

std::shared_ptr<Backend> Lookup(const std::string &name, bool *ok) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  for (auto &b : g_registry)
    if (b->Name() == name) {
      if (ok) *ok = true;
      return b;
    }
  if (ok) *ok = false;
  return nullptr;
}

std::shared_ptr<Backend> Default() {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  for (auto &b : g_registry)
    if (b->Class() == CorrectnessClass::Reference) return b;
  return g_registry.empty() ? nullptr : g_registry.front();
}

std::shared_ptr<Backend> Pick(const std::string &name) {
  if (!name.empty()) {
    bool ok = false;
    auto b = Lookup(name, &ok);
    if (ok) return b;
  }
  return Default();
}

bool RequireReference(const Backend *b) {
  return b != nullptr && b->Class() == CorrectnessClass::Reference;
}

bool RegisterRocm() {
  std::shared_ptr<Backend> be;
  try {
    be = std::make_shared<RocmBackend>();
  } catch (const std::runtime_error &) {
    return false;  // no gfx950 device: register nothing (cuda.go:215-217)
  }
  Register(be);
  return true;
}

void ResetRegistry() {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  g_registry.clear();
}

// ---- model-level seams ----

Q6KWeight UploadQ6K(const uint8_t *raw, size_t len, int out, int in) {
  Q6KWeight w;
  if (!raw || out <= 0 || in <= 0 || in % 256) return w;
  if (len < (size_t)out * (in / 256) * 210) return w;
  w.ptr = fhip_q6k_upload(raw, out, in);
  if (w.ptr) {
    w.Out = out;
    w.In = in;
  }
  return w;
}

void FreeQ6K(Q6KWeight &w) {
  if (w.ptr) fhip_free(w.ptr);
  w = Q6KWeight{};
}

void Q6KMatRows(const Q6KWeight &w, const Tensor &X, Tensor &Y, int P) {
  const DeviceBuffer *xb = X.device(), *yb = Y.device();
  if (!w || !xb || !yb || X.Numel() != (long long)P * w.In || Y.Numel() != (long long)P * w.Out)
    throw std::invalid_argument("compute: Q6KMatRows shape or residency mismatch");
  check("fhip_q6k_matmul_f32", fhip_q6k_matmul_f32(w.ptr, (const float *)xb->ptr,
                                                   (float *)yb->ptr, w.Out, w.In, P));
}

namespace {
bool mlp_shapes(const Tensor &gate, const Tensor &up, int down_out, int down_in, const Tensor &x,
                const Tensor &y, int P) {
  if (gate.dtype != Dtype::Q4_K || up.dtype != Dtype::Q4_K || gate.shape.size() != 2 ||
      up.shape.size() != 2 || !gate.device() || !up.device() || !x.device() || !y.device())
    return false;
  const int I = gate.shape[0], H = gate.shape[1];
  if (up.shape[0] != I || up.shape[1] != H || down_in != I || down_out != H) return false;
  return P >= 1 && P <= 4 && x.Numel() >= (long long)P * H && y.Numel() >= (long long)P * H;
}
}  // namespace

bool FusedMLP(const Tensor &gate, const Tensor &up, const Tensor &down, const Tensor &x,
              Tensor &y, int P) {
  if (down.dtype != Dtype::Q4_K || down.shape.size() != 2 || !down.device()) return false;
  if (!mlp_shapes(gate, up, down.shape[0], down.shape[1], x, y, P)) return false;
  check("fhip_q4k_mlp_f32",
        fhip_q4k_mlp_f32(gate.device()->ptr, up.device()->ptr, down.device()->ptr,
                         (const float *)x.device()->ptr, (float *)y.device()->ptr, gate.shape[1],
                         gate.shape[0], P));
  return true;
}

bool FusedMLPQ6Down(const Tensor &gate, const Tensor &up, const Q6KWeight &down,
                    const Tensor &x, Tensor &y, int P) {
  if (!down || !mlp_shapes(gate, up, down.Out, down.In, x, y, P)) return false;
  check("fhip_q4k_mlp_q6down_f32",
        fhip_q4k_mlp_q6down_f32(gate.device()->ptr, up.device()->ptr, down.ptr,
                                (const float *)x.device()->ptr, (float *)y.device()->ptr,
                                gate.shape[1], gate.shape[0], P));
  return true;
}

}  // namespace compute
}  // namespace fak
