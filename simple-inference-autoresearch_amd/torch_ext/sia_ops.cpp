// _sia_ops: the thin PyTorch-ROCm extension between the Python drop-ins and
// the C ABI of libsia_attention.so (include/sia_attention.h).
//
// Each op checks that every tensor lives on q's (or k's) GPU, describes the
// tensors for the C ABI, takes outputs and split-K workspace from torch's
// caching allocator, and calls the entry point on torch's current HIP stream
// of that device.  A non-zero status becomes the Python exception the
// reference's wrappers would raise: ValueError for an invalid argument,
// NotImplementedError for an unsupported but valid one, SiaError (a
// RuntimeError) for a launch or device failure.  Nothing here computes: the
// kernels are the library's.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <mutex>
#include <tuple>
#include <unordered_map>

#include "sia_attention.h"

namespace py = pybind11;
using at::Tensor;
using OptT = std::optional<Tensor>;

namespace {

PyObject* g_sia_error = nullptr;   // Python class for launch/device failures (a new reference, kept)

[[noreturn]] void raise_status(int rc) {
  const char* msg = sia_last_error_message();
  std::string text = std::string(sia_status_string(rc)) + (msg && *msg ? std::string(": ") + msg : "");
  if (rc == SIA_ERR_INVALID_ARGUMENT) throw py::value_error(text);
  PyObject* cls = rc == SIA_ERR_UNSUPPORTED ? PyExc_NotImplementedError
                  : g_sia_error == nullptr  ? PyExc_RuntimeError
                                            : g_sia_error;
  PyErr_SetString(cls, text.c_str());
  throw py::error_already_set();
}

inline void check(int rc) {
  if (rc != SIA_OK) raise_status(rc);
}

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return SIA_F16;
    case at::kBFloat16: return SIA_BF16;
    case at::kFloat: return SIA_F32;
    case at::kChar: return SIA_I8;
    case at::kInt: return SIA_I32;
    case at::kLong: return SIA_I64;
    case at::kByte: return SIA_U8;
    default: throw py::value_error(std::string("dtype ") + c10::toString(t) + " is not supported by the attention kernels");
  }
}

// Descriptor of a tensor that must live on `dev` (a host tensor would hand a
// host address to the kernels).
sia_tensor desc(const Tensor& t, const at::Device& dev, const char* name) {
  if (t.device() != dev)
    throw py::value_error(std::string(name) + " is on " + t.device().str() + "; every tensor of the call must be on " +
                          dev.str());
  if (t.dim() > SIA_MAX_DIMS)
    throw py::value_error(std::string(name) + " has " + std::to_string(t.dim()) + " dims; at most 5 are supported");
  sia_tensor d;
  d.data = t.data_ptr();
  d.dtype = dtype_code(t.scalar_type());
  d.ndim = (int32_t)t.dim();
  for (int i = 0; i < d.ndim; ++i) {
    d.shape[i] = t.size(i);
    d.stride[i] = t.stride(i);
  }
  return d;
}

// Descriptor or NULL for an optional tensor.
struct OptDesc {
  sia_tensor d;
  bool set = false;
  OptDesc(const OptT& t, const at::Device& dev, const char* name) {
    if (t.has_value()) {
      d = desc(*t, dev, name);
      set = true;
    }
  }
  const sia_tensor* ptr() const { return set ? &d : nullptr; }
};

at::Device gpu_of(const Tensor& t, const char* name) {
  if (!t.is_cuda())
    throw py::value_error(std::string("the attention kernels run on the GPU: ") + name +
                          " must be a CUDA (HIP) tensor");
  return t.device();
}

void* stream_of(const at::Device& dev) { return (void*)c10::hip::getCurrentHIPStream(dev.index()).stream(); }

// Workspace sizes by geometry (the C ABI's answer depends on the device's CU count).
std::mutex g_mu;
std::unordered_map<uint64_t, size_t> g_ws;

size_t decode_ws_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int dev) {
  const uint64_t key = ((uint64_t)B << 40) ^ ((uint64_t)Hq << 28) ^ ((uint64_t)Hkv << 16) ^ ((uint64_t)D << 4) ^
                       (uint64_t)dev;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_ws.find(key);
    if (it != g_ws.end()) return it->second;
  }
  size_t n = 0;
  check(sia_decode_workspace_size(B, Hq, Hkv, D, &n));
  std::lock_guard<std::mutex> lock(g_mu);
  g_ws[key] = n;
  return n;
}

enum DecodeKind { kContig = 0, kContigInt8 = 1, kGqaInt8 = 2, kPaged = 3, kPagedInt8 = 4 };

// One decode call (q (B, Hq, 1, D)) -> out (B, 1, Hq, D) in q's dtype.
Tensor decode(int64_t kind, const Tensor& q, const Tensor& k, const Tensor& v, const OptT& k_scale,
              const OptT& v_scale, const OptT& block_table, const Tensor& kv_len, int64_t page_size, double sm_scale,
              int64_t tiles_per_split, int64_t begin_event, int64_t end_event) {
  const at::Device dev = gpu_of(q, "q");
  const c10::DeviceGuard guard(dev);
  if (q.dim() != 4) throw py::value_error("q must be (B, Hq, 1, D)");
  if (k.dim() != 4) throw py::value_error("k must have 4 dims");
  const int64_t B = q.size(0), Hq = q.size(1), D = q.size(3), Hkv = k.size(1);
  // an empty batch has nothing to compute (the reference's launch over a
  // grid of B * Hq programs does nothing either)
  if (B == 0) return at::empty({0, 1, Hq, D}, q.options());
  const sia_tensor dq = desc(q, dev, "q"), dk = desc(k, dev, "k"), dv = desc(v, dev, "v");
  const sia_tensor dl = desc(kv_len, dev, "kv_len");
  const OptDesc dks(k_scale, dev, "k_scale"), dvs(v_scale, dev, "v_scale"), dbt(block_table, dev, "block_table");
  Tensor out = at::empty({B, 1, Hq, D}, q.options());
  const sia_tensor dout = desc(out, dev, "out");
  const size_t ws_bytes = decode_ws_bytes(B, Hq, Hkv, D, dev.index());
  Tensor ws = at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte));
  sia_decode_options opts;
  memset(&opts, 0, sizeof(opts));
  opts.tiles_per_split = (int32_t)tiles_per_split;
  opts.main_begin_event = (void*)begin_event;
  opts.main_end_event = (void*)end_event;
  const sia_decode_options* po = (tiles_per_split || begin_event || end_event) ? &opts : nullptr;
  void* s = stream_of(dev);
  const float sc = (float)sm_scale;
  int rc;
  switch (kind) {
    case kContig:
      rc = sia_attention_flash_decode(&dq, &dk, &dv, &dl, sc, &dout, ws.data_ptr(), ws_bytes, po, s);
      break;
    case kContigInt8:
      rc = sia_attention_flash_decode_int8(&dq, &dk, &dv, dks.ptr(), dvs.ptr(), &dl, sc, &dout, ws.data_ptr(),
                                           ws_bytes, po, s);
      break;
    case kGqaInt8:
      rc = sia_gqa_int8_flash_decode(&dq, &dk, &dv, dks.ptr(), dvs.ptr(), &dl, sc, &dout, ws.data_ptr(), ws_bytes,
                                     po, s);
      break;
    case kPaged:
      rc = sia_paged_attention_flash_decode(&dq, &dk, &dv, dbt.ptr(), &dl, (int32_t)page_size, sc, &dout,
                                            ws.data_ptr(), ws_bytes, po, s);
      break;
    case kPagedInt8:
      rc = sia_paged_gqa_int8_flash_decode(&dq, &dk, &dv, dks.ptr(), dvs.ptr(), dbt.ptr(), &dl, (int32_t)page_size,
                                           sc, &dout, ws.data_ptr(), ws_bytes, po, s);
      break;
    default:
      throw py::value_error("unknown decode kind");
  }
  check(rc);
  return out;
}

// A prefill operand as the kernels read it: in place when head_dim is
// contiguous, rows are 16-byte aligned and the rows of one 64-key block lie
// within 32-bit offsets; any other view is copied.
Tensor readable(const Tensor& t) {
  if (t.dim() < 2) return t;
  const int64_t es = t.element_size();
  bool ok = t.stride(-1) == 1 && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
  for (int64_t i = 0; ok && i < t.dim() - 1; ++i) ok = (t.stride(i) * es) % 16 == 0;
  if (ok && t.size(-2) > 1) {
    const int64_t row = t.stride(-2) * es;
    ok = t.size(-1) * es <= row && row < (int64_t(1) << 31) / 64;
  }
  return ok ? t : t.contiguous();
}

// The prefill takes no workspace for fp32 (vector-ALU path) and for float16
// at head_dim 32-128, whose V is read in place; otherwise V is repacked into
// f16 block images in the workspace.  (The same rule as v_in_place in
// csrc/capi_prefill.cpp; were they to differ, the library would refuse the
// call with SIA_ERR_WORKSPACE rather than touch memory it was not given.)
bool v_in_place(const Tensor& q) {
  const int64_t D = q.size(-1);
  return q.scalar_type() == at::kFloat || (q.scalar_type() == at::kHalf && D >= 32 && D <= 128);
}

// Causal / full attention (q (B, Hq, Tq, D)) -> (B, Hq, Tq, D) or token-major (B, Tq, Hq, D).
Tensor prefill(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, bool causal, double sm_scale,
               bool out_token_major) {
  const at::Device dev = gpu_of(q_in, "q");
  const c10::DeviceGuard guard(dev);
  if (q_in.dim() != 4 || k_in.dim() != 4) throw py::value_error("q, k and v must have 4 dims");
  const Tensor q = readable(q_in), k = readable(k_in), v = readable(v_in);
  const int64_t B = q.size(0), Hq = q.size(1), Tq = q.size(2), D = q.size(3);
  const int64_t Hkv = k.size(1), Tk = k.size(2);
  const sia_tensor dq = desc(q, dev, "q"), dk = desc(k, dev, "k"), dv = desc(v, dev, "v");
  Tensor out = out_token_major ? at::empty({B, Tq, Hq, D}, q.options()) : at::empty({B, Hq, Tq, D}, q.options());
  const Tensor view = out_token_major ? out.transpose(1, 2) : out;
  const sia_tensor dout = desc(view, dev, "out");
  size_t ws_bytes = 0;
  if (!v_in_place(q)) check(sia_prefill_workspace_size(B, Hkv, Tk, D, &ws_bytes));
  Tensor ws = ws_bytes > 0 ? at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte)) : Tensor();
  check(sia_attention_flash_fwd(&dq, &dk, &dv, causal ? 1 : 0, (float)sm_scale, &dout,
                                ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(dev)));
  return out;
}

// prefill with q rotated at load: q (B, Hq, Tq, D) un-rotated, k rotated.
Tensor prefill_rope(const Tensor& q_in, const Tensor& k_in, const Tensor& v_in, const Tensor& cos, const Tensor& sin,
                    bool interleaved, const OptT& start_pos, int64_t start_offset, bool causal, double sm_scale,
                    bool out_token_major) {
  const at::Device dev = gpu_of(q_in, "q");
  const c10::DeviceGuard guard(dev);
  if (q_in.dim() != 4 || k_in.dim() != 4) throw py::value_error("q, k and v must have 4 dims");
  const Tensor q = readable(q_in), k = readable(k_in), v = readable(v_in);
  const int64_t B = q.size(0), Hq = q.size(1), Tq = q.size(2), D = q.size(3);
  const int64_t Hkv = k.size(1), Tk = k.size(2);
  const sia_tensor dq = desc(q, dev, "q"), dk = desc(k, dev, "k"), dv = desc(v, dev, "v"),
                   dc = desc(cos, dev, "cos"), dsn = desc(sin, dev, "sin");
  const OptDesc dsp(start_pos, dev, "start_pos");
  Tensor out = out_token_major ? at::empty({B, Tq, Hq, D}, q.options()) : at::empty({B, Hq, Tq, D}, q.options());
  const Tensor view = out_token_major ? out.transpose(1, 2) : out;
  const sia_tensor dout = desc(view, dev, "out");
  size_t ws_bytes = 0;
  if (!v_in_place(q)) check(sia_prefill_workspace_size(B, Hkv, Tk, D, &ws_bytes));
  Tensor ws = ws_bytes > 0 ? at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte)) : Tensor();
  check(sia_attention_flash_fwd_rope(&dq, &dk, &dv, &dc, &dsn, interleaved ? 1 : 0, dsp.ptr(), (int32_t)start_offset,
                                     causal ? 1 : 0, (float)sm_scale, &dout, ws_bytes > 0 ? ws.data_ptr() : nullptr,
                                     ws_bytes,
                                     stream_of(dev)));
  return out;
}

std::tuple<Tensor, Tensor> quantize_kv_int8(const Tensor& x, bool scale_f32) {
  const at::Device dev = gpu_of(x, "x");
  const c10::DeviceGuard guard(dev);
  Tensor xi = at::empty(x.sizes(), x.options().dtype(at::kChar));
  std::vector<int64_t> ss(x.sizes().begin(), x.sizes().end());
  if (!ss.empty()) ss.pop_back();
  Tensor scale = at::empty(ss, x.options().dtype(scale_f32 ? at::kFloat : at::kHalf));
  if (x.numel() == 0 && x.dim() >= 1) return {xi, scale};   // nothing to quantise (empty tensors have no data)
  const sia_tensor dx = desc(x, dev, "x");
  const sia_tensor dxi = desc(xi, dev, "out"), ds = desc(scale, dev, "scale");
  check(sia_quantize_kv_int8(&dx, &dxi, &ds, stream_of(dev)));
  return {xi, scale};
}

void kv_write(const Tensor& k, const OptT& v, const Tensor& k_dst, const OptT& v_dst, const OptT& k_scale_dst,
              const OptT& v_scale_dst, const OptT& block_table, const OptT& start_pos, int64_t start_offset,
              int64_t page_size) {
  const at::Device dev = gpu_of(k, "k");
  const c10::DeviceGuard guard(dev);
  if (k.numel() == 0 && k.dim() == 4) return;   // no tokens to write
  const sia_tensor dk = desc(k, dev, "k"), dkd = desc(k_dst, dev, "k_dst");
  const OptDesc dv(v, dev, "v"), dvd(v_dst, dev, "v_dst"), dks(k_scale_dst, dev, "k_scale_dst"),
      dvs(v_scale_dst, dev, "v_scale_dst"), dbt(block_table, dev, "block_table"), dsp(start_pos, dev, "start_pos");
  check(sia_kv_write(&dk, dv.ptr(), &dkd, dvd.ptr(), dks.ptr(), dvs.ptr(), dbt.ptr(), dsp.ptr(), (int32_t)start_offset,
                     (int32_t)page_size, stream_of(dev)));
}

OptT rope_kv_write(const OptT& q, const Tensor& k, const OptT& v, const Tensor& cos, const Tensor& sin,
                   const Tensor& k_dst, const OptT& v_dst, const OptT& k_scale_dst, const OptT& v_scale_dst,
                   const OptT& block_table, const OptT& start_pos, int64_t start_offset, int64_t page_size,
                   bool interleaved, const OptT& q_out) {
  const at::Device dev = gpu_of(k, "k");
  const c10::DeviceGuard guard(dev);
  OptT qo = q_out;
  if (q.has_value() && !qo.has_value()) qo = at::empty(q->sizes(), q->options());
  if (k.numel() == 0 && k.dim() == 4 && (!q.has_value() || q->numel() == 0)) return qo;   // no tokens
  const sia_tensor dk = desc(k, dev, "k"), dc = desc(cos, dev, "cos"), dsn = desc(sin, dev, "sin"),
                   dkd = desc(k_dst, dev, "k_dst");
  const OptDesc dq(q, dev, "q"), dv(v, dev, "v"), dqo(qo, dev, "q_out"), dvd(v_dst, dev, "v_dst"),
      dks(k_scale_dst, dev, "k_scale_dst"), dvs(v_scale_dst, dev, "v_scale_dst"), dbt(block_table, dev, "block_table"),
      dsp(start_pos, dev, "start_pos");
  check(sia_rope_kv_write(dq.ptr(), &dk, dv.ptr(), &dc, &dsn, interleaved ? 1 : 0, dqo.ptr(), &dkd, dvd.ptr(),
                          dks.ptr(), dvs.ptr(), dbt.ptr(), dsp.ptr(), (int32_t)start_offset, (int32_t)page_size,
                          stream_of(dev)));
  return qo;
}

// A (B, T, H, D) view whose B*T rows sit one stride apart (head_dim
// unit-stride, heads D apart), as sia_rope_qk reads it; other views are
// copied first (kernels/rope_kernel.py:216-235 does the same).
bool rows_flattenable(const Tensor& x) {
  if (x.dim() != 4) return true;   // the C ABI reports the shape error
  const int64_t T = x.size(1), H = x.size(2), D = x.size(3);
  if (x.stride(3) != 1 || (H > 1 && x.stride(2) != D)) return false;
  return T == 1 || x.size(0) == 1 || x.stride(0) == T * x.stride(1);
}

std::tuple<Tensor, Tensor> rope_qk(const Tensor& q_in, const Tensor& k_in, const Tensor& cos, const Tensor& sin,
                                   bool interleaved) {
  const at::Device dev = gpu_of(q_in, "q");
  const c10::DeviceGuard guard(dev);
  const Tensor q = rows_flattenable(q_in) ? q_in : q_in.contiguous();
  const Tensor k = rows_flattenable(k_in) ? k_in : k_in.contiguous();
  const sia_tensor dq = desc(q, dev, "q"), dk = desc(k, dev, "k"), dc = desc(cos, dev, "cos"),
                   dsn = desc(sin, dev, "sin");
  Tensor qo = at::empty(q.sizes(), q.options());
  Tensor ko = at::empty(k.sizes(), k.options());
  if (q.numel() == 0 && k.numel() == 0 && q.dim() == 4 && k.dim() == 4) return {qo, ko};   // no tokens
  const sia_tensor dqo = desc(qo, dev, "q_out"), dko = desc(ko, dev, "k_out");
  check(sia_rope_qk(&dq, &dk, &dc, &dsn, interleaved ? 1 : 0, &dqo, &dko, stream_of(dev)));
  return {qo, ko};
}

}  // namespace

PYBIND11_MODULE(_sia_ops, m) {
  m.doc() = "Thin torch bindings of libsia_attention.so (include/sia_attention.h)";
  m.def("set_error_class", [](py::object cls) {
    PyObject* old = g_sia_error;
    g_sia_error = cls.inc_ref().ptr();
    Py_XDECREF(old);
  });
  m.def("abi_version", []() { return sia_abi_version(); });
  m.def("decode_workspace_size", [](int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
    size_t n = 0;
    check(sia_decode_workspace_size(B, Hq, Hkv, D, &n));
    return n;
  });
  m.def("prefill_workspace_size", [](int64_t B, int64_t Hkv, int64_t Tk, int64_t D) {
    size_t n = 0;
    check(sia_prefill_workspace_size(B, Hkv, Tk, D, &n));
    return n;
  });
  m.def("decode", &decode);
  m.def("prefill", &prefill);
  m.def("prefill_rope", &prefill_rope);
  m.def("quantize_kv_int8", &quantize_kv_int8);
  m.def("kv_write", &kv_write);
  m.def("rope_kv_write", &rope_kv_write);
  m.def("rope_qk", &rope_qk);
}
