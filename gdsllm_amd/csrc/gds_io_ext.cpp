// gds_io_ext — the Python module the reference's model code imports
// (runtime/gds_bindings.cpp:516-615), rebuilt as a PyTorch-ROCm extension over
// the gdsllm_amd C ABI.  Same function names, argument names and defaults,
// output shapes and RuntimeError messages for the compute ops; the cuFile
// loader is replaced by HBM-resident buffers filled with pread + hipMemcpy.
//
// This file holds no kernels: every op validates its tensors, resolves the
// current HIP stream of the target device and calls one extern "C" entry
// point of libgdsllm_amd.so, converting a non-zero status into RuntimeError.

#include <torch/extension.h>
#include <c10/hip/HIPStream.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "gdsllm_amd.h"

namespace py = pybind11;

namespace {

void check(int rc, const std::string& where) {
    if (rc != GDSLLM_OK) {
        std::string msg = gdsllm_last_error();
        if (msg.empty()) msg = "error code " + std::to_string(rc);
        throw std::runtime_error(where + ": " + msg);
    }
}

// Makes `device_id` the current HIP device for the scope (the library plans
// launch geometry for the current device) and resolves its current stream.
// Used as a named guard or as a temporary inside the full expression of the
// call it serves.
class OnDevice {
  public:
    explicit OnDevice(int device_id) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != device_id) {
            if (hipSetDevice(device_id) != hipSuccess)
                throw std::runtime_error("cannot make cuda:" + std::to_string(device_id) + " the current device");
            restore_ = prev_ >= 0;
        }
        stream_ = c10::hip::getCurrentHIPStream(device_id).stream();
    }
    ~OnDevice() {
        if (restore_) (void)hipSetDevice(prev_);
    }
    OnDevice(const OnDevice&) = delete;
    OnDevice& operator=(const OnDevice&) = delete;
    void* stream() const { return stream_; }

  private:
    int prev_ = -1;
    bool restore_ = false;
    void* stream_ = nullptr;
};

// Device buffer with the GdsBufferHandle surface (runtime/gds_bindings.cpp:51-76):
// size / device_id / registered.  Either owns a hipMalloc allocation, or wraps
// the storage of a device tensor it keeps alive (for synthetic weights).
class GdsBufferHandle {
  public:
    GdsBufferHandle(size_t size, int device_id) : device_id_(device_id) {
        size_t rounded = 0;
        check(gdsllm_buffer_alloc(size, device_id, &ptr_, &rounded), "gds_alloc");
        size_ = rounded;
        owned_ = true;
    }
    explicit GdsBufferHandle(const torch::Tensor& t) : keep_(t) {
        if (!t.is_cuda()) throw std::runtime_error("GdsBufferHandle.from_tensor: tensor must be on a GPU");
        if (!t.is_contiguous()) throw std::runtime_error("GdsBufferHandle.from_tensor: tensor must be contiguous");
        ptr_ = t.data_ptr();
        size_ = static_cast<size_t>(t.numel()) * t.element_size();
        device_id_ = t.get_device();
    }
    ~GdsBufferHandle() {
        if (owned_ && ptr_) gdsllm_buffer_free(ptr_, device_id_);
    }
    GdsBufferHandle(const GdsBufferHandle&) = delete;
    GdsBufferHandle& operator=(const GdsBufferHandle&) = delete;

    void* dev_ptr() const { return ptr_; }
    size_t size() const { return size_; }
    int device_id() const { return device_id_; }
    bool registered() const { return false; }  // no cuFile registration on this platform
    int64_t data_ptr() const { return reinterpret_cast<int64_t>(ptr_); }

  private:
    void* ptr_ = nullptr;
    size_t size_ = 0;
    int device_id_ = 0;
    bool owned_ = false;
    torch::Tensor keep_;
};
using Handle = std::shared_ptr<GdsBufferHandle>;

bool g_initialized = false;

void init() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        throw std::runtime_error("init: no HIP device available");
    g_initialized = true;
}
void shutdown() { g_initialized = false; }
bool is_driver_open() { return g_initialized; }

torch::Dtype parse_dtype(const std::string& s) {
    if (s == "float16" || s == "half") return torch::kFloat16;
    if (s == "float32" || s == "float") return torch::kFloat32;
    if (s == "bfloat16") return torch::kBFloat16;
    if (s == "int8") return torch::kInt8;
    if (s == "int32" || s == "int") return torch::kInt32;
    if (s == "uint32") return torch::kUInt32;
    if (s == "uint8") return torch::kUInt8;
    throw std::runtime_error("Unsupported dtype: " + s);
}

const char* at_offset(const Handle& h, int64_t offset) {
    return static_cast<const char*>(h->dev_ptr()) + offset;
}

void check_handle(const Handle& h, const char* where) {
    if (!h || !h->dev_ptr()) throw std::runtime_error(std::string(where) + ": invalid buffer handle");
}

void check_range(const Handle& h, int64_t offset, int64_t bytes, const char* where) {
    if (offset < 0 || bytes < 0 || static_cast<uint64_t>(offset) + static_cast<uint64_t>(bytes) > h->size())
        throw std::runtime_error(std::string(where) + ": byte range [" + std::to_string(offset) + ", " +
                                 std::to_string(offset + bytes) + ") exceeds buffer of " +
                                 std::to_string(h->size()) + " bytes");
}

torch::TensorOptions fp16_on(int device_id) {
    return torch::TensorOptions().dtype(torch::kFloat16).device(torch::kCUDA, device_id);
}

void check_x(const torch::Tensor& x, int device_id, const char* where) {
    if (!x.is_cuda() || x.get_device() != device_id)
        throw std::runtime_error(std::string(where) + ": x must be on the weight buffer's device (cuda:" +
                                 std::to_string(device_id) + ")");
    if (x.scalar_type() != torch::kFloat16) throw std::runtime_error(std::string(where) + ": x must be float16");
}

// ---- loaders (runtime/gds_bindings.cpp:95-247) --------------------------------

Handle load_file(const std::string& path, int64_t size_bytes, int device_id) {
    auto h = std::make_shared<GdsBufferHandle>(size_bytes, device_id);
    int64_t got = 0;
    check(gdsllm_buffer_read_file(h->dev_ptr(), h->size(), path.c_str(), size_bytes, 0, 0, device_id, &got),
          "py_load_file");
    if (got < size_bytes)
        throw std::runtime_error("py_load_file: expected " + std::to_string(size_bytes) + " bytes, got " +
                                 std::to_string(got));
    return h;
}

Handle load_file_region(const std::string& path, int64_t size_bytes, int64_t file_offset, int device_id) {
    auto h = std::make_shared<GdsBufferHandle>(size_bytes, device_id);
    int64_t got = 0;
    check(gdsllm_buffer_read_file(h->dev_ptr(), h->size(), path.c_str(), size_bytes, file_offset, 0, device_id,
                                  &got),
          "py_load_file_region");
    if (got < size_bytes)
        throw std::runtime_error("py_load_file_region: expected " + std::to_string(size_bytes) + " bytes, got " +
                                 std::to_string(got));
    return h;
}

py::tuple load_expert(const std::string& path, int64_t w_off, int64_t w_size, int64_t s_off, int64_t s_size,
                      int64_t b_off, int64_t b_size, int device_id) {
    auto h = std::make_shared<GdsBufferHandle>(w_size + s_size + b_size, device_id);
    const struct {
        int64_t file_off, size, buf_off;
        const char* what;
    } parts[3] = {{w_off, w_size, 0, "py_load_expert: short read on weight"},
                  {s_off, s_size, w_size, "py_load_expert: short read on scale"},
                  {b_off, b_size, w_size + s_size, "py_load_expert: short read on bias"}};
    for (const auto& p : parts) {
        int64_t got = 0;
        check(gdsllm_buffer_read_file(h->dev_ptr(), h->size(), path.c_str(), p.size, p.file_off, p.buf_off,
                                      device_id, &got),
              "py_load_expert");
        if (got < p.size) throw std::runtime_error(p.what);
    }
    return py::make_tuple(h, static_cast<int64_t>(0), w_size, w_size + s_size);
}

torch::Tensor view_tensor(const Handle& h, std::vector<int64_t> shape, const std::string& dtype, int64_t offset) {
    if (!h || !h->dev_ptr()) throw std::runtime_error("py_view_tensor: invalid buffer handle");
    const auto dt = parse_dtype(dtype);
    int64_t n = 1;
    for (auto s : shape) n *= s;
    check_range(h, offset, n * static_cast<int64_t>(c10::elementSize(dt)), "py_view_tensor");
    Handle ref = h;  // the deleter keeps the buffer alive as long as the view
    return torch::from_blob(static_cast<char*>(h->dev_ptr()) + offset, shape, [ref](void*) {},
                            torch::TensorOptions().dtype(dt).device(torch::kCUDA, h->device_id()));
}

torch::Tensor load_tensor(const std::string& path, std::vector<int64_t> shape, const std::string& dtype,
                          int64_t file_offset, int64_t size_bytes, int device_id) {
    const auto dt = parse_dtype(dtype);
    if (size_bytes <= 0) {
        int64_t n = 1;
        for (auto s : shape) n *= s;
        size_bytes = n * static_cast<int64_t>(c10::elementSize(dt));
    }
    auto h = std::make_shared<GdsBufferHandle>(size_bytes, device_id);
    int64_t got = 0;
    check(gdsllm_buffer_read_file(h->dev_ptr(), h->size(), path.c_str(), size_bytes, file_offset, 0, device_id,
                                  &got),
          "py_load_tensor");
    if (got < size_bytes)
        throw std::runtime_error("py_load_tensor: expected " + std::to_string(size_bytes) + " bytes, got " +
                                 std::to_string(got));
    return view_tensor(h, shape, dtype, 0);
}

// ---- compute ops (runtime/gds_bindings.cpp:255-512) ----------------------------

int64_t gguf_block_bytes(const std::string& t, const char* where) {
    if (t == "q4_0") return 18;
    if (t == "q8_0") return 34;
    throw std::runtime_error(std::string(where) + ": unsupported type '" + t + "'");
}

torch::Tensor dequant_gguf(const Handle& h, std::vector<int64_t> shape, const std::string& gguf_type,
                           int64_t offset, c10::optional<torch::Tensor> output) {
    check_handle(h, "py_dequant_gguf");
    int64_t n = 1;
    for (auto s : shape) n *= s;
    if (n % 32 != 0)
        throw std::runtime_error("py_dequant_gguf: total elements must be a multiple of 32 (block size), got " +
                                 std::to_string(n));
    const int64_t blocks = n / 32;
    const int64_t bb = gguf_block_bytes(gguf_type, "py_dequant_gguf");
    check_range(h, offset, blocks * bb, "py_dequant_gguf");
    torch::Tensor out;
    if (output.has_value()) {
        out = output.value();
        if (out.numel() < n)
            throw std::runtime_error("py_dequant_gguf: scratch buffer too small (" + std::to_string(out.numel()) +
                                     " < " + std::to_string(n) + ")");
        if (out.scalar_type() != torch::kFloat16 || !out.is_cuda() || !out.is_contiguous())
            throw std::runtime_error("py_dequant_gguf: scratch must be a contiguous float16 GPU tensor");
        out = out.flatten().slice(0, 0, n).view(shape);
    } else {
        out = torch::empty(shape, fp16_on(h->device_id()));
    }
    const OnDevice on(h->device_id());
    void* s = on.stream();
    const int rc = gguf_type == "q4_0" ? gdsllm_dequant_q4_0(at_offset(h, offset), out.data_ptr(), blocks, s)
                                       : gdsllm_dequant_q8_0(at_offset(h, offset), out.data_ptr(), blocks, s);
    check(rc, "py_dequant_gguf");
    return out;
}

// Embedding rows of a GGUF table [vocab, hidden] for token_ids (any shape,
// int64/int32, on the buffer's device): output token_ids.shape + [hidden]
// fp16, the rows F.embedding would take from the dequantized table
// (runtime/scheduler.py:22-35) without dequantizing the rest of it.
torch::Tensor embed_gguf(const Handle& h, torch::Tensor token_ids, std::vector<int64_t> shape,
                         const std::string& gguf_type, int64_t offset) {
    const char* where = "embed_gguf";
    check_handle(h, where);
    if (shape.size() != 2) throw std::runtime_error("embed_gguf: shape must be [vocab, hidden]");
    const int64_t vocab = shape[0], hidden = shape[1];
    const int64_t bb = gguf_block_bytes(gguf_type, where);
    if (hidden % 32 != 0) throw std::runtime_error("embed_gguf: hidden must be a multiple of 32");
    check_range(h, offset, vocab * (hidden / 32) * bb, where);
    if (!token_ids.is_cuda() || token_ids.get_device() != h->device_id())
        throw std::runtime_error("embed_gguf: token_ids must be on the weight buffer's device");
    auto ids = token_ids.to(torch::kInt64).contiguous().view(-1);
    std::vector<int64_t> out_shape(token_ids.sizes().begin(), token_ids.sizes().end());
    out_shape.push_back(hidden);
    auto out = torch::empty(out_shape, fp16_on(h->device_id()));
    const OnDevice on(h->device_id());
    void* s = on.stream();
    const int64_t n = ids.numel();
    for (int64_t t = 0; t < n; t += 65535) {
        const int64_t c = std::min<int64_t>(65535, n - t);
        const auto* ip = ids.data_ptr<int64_t>() + t;
        auto* op = static_cast<uint16_t*>(out.data_ptr()) + t * hidden;
        const int rc = gguf_type == "q4_0" ? gdsllm_embed_q4_0(at_offset(h, offset), ip, c, vocab, hidden, op, s)
                                           : gdsllm_embed_q8_0(at_offset(h, offset), ip, c, vocab, hidden, op, s);
        check(rc, where);
    }
    return out;
}

// x: [in_dim] / [1, in_dim] (the reference's contract) or [B, in_dim], B <= 8.
// Returns [B, out_dim]; B = 1 reproduces the reference's [1, out_dim].
torch::Tensor fused_dequant_gemv(const Handle& h, torch::Tensor x, std::vector<int64_t> weight_shape,
                                 const std::string& gguf_type, int64_t offset) {
    check_handle(h, "py_fused_dequant_gemv");
    if (weight_shape.size() != 2)
        throw std::runtime_error("py_fused_dequant_gemv: weight_shape must be [out_dim, in_dim]");
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    if (in_dim % 32 != 0)
        throw std::runtime_error("py_fused_dequant_gemv: in_dim must be a multiple of 32, got " +
                                 std::to_string(in_dim));
    const int64_t bb = gguf_block_bytes(gguf_type, "py_fused_dequant_gemv");
    torch::Tensor xf = x.contiguous();
    const int64_t numel = xf.numel();
    int64_t batch = 1;
    if (numel != in_dim) {
        if (in_dim > 0 && numel % in_dim == 0 && numel / in_dim <= 8 && xf.dim() >= 2 && xf.size(-1) == in_dim)
            batch = numel / in_dim;
        else
            throw std::runtime_error("py_fused_dequant_gemv: input size " + std::to_string(numel) +
                                     " != in_dim " + std::to_string(in_dim));
    }
    check_x(xf, h->device_id(), "py_fused_dequant_gemv");
    check_range(h, offset, out_dim * (in_dim / 32) * bb, "py_fused_dequant_gemv");
    torch::Tensor out = torch::empty({batch, out_dim}, fp16_on(h->device_id()));
    const OnDevice on(h->device_id());
    void* s = on.stream();
    const int rc = gguf_type == "q4_0"
                       ? gdsllm_fused_q4_0_gemv(at_offset(h, offset), xf.data_ptr(), out.data_ptr(), out_dim, in_dim,
                                                batch, in_dim, out_dim, s)
                       : gdsllm_fused_q8_0_gemv(at_offset(h, offset), xf.data_ptr(), out.data_ptr(), out_dim, in_dim,
                                                batch, in_dim, out_dim, s);
    check(rc, "py_fused_dequant_gemv");
    return out;
}

struct AffinePtrs {
    const char *w, *s, *b;
};

AffinePtrs affine_ptrs(const Handle& h, int64_t rows, int64_t in_dim, int64_t w_off, int64_t s_off, int64_t b_off,
                       int64_t group_size, const char* where) {
    if (group_size <= 0) throw std::runtime_error(std::string(where) + ": group_size must be positive");
    if (in_dim % 8 != 0)
        throw std::runtime_error(std::string(where) + ": in_dim must be a multiple of 8, got " + std::to_string(in_dim));
    check_range(h, w_off, rows * (in_dim / 8) * 4, where);
    const int64_t groups = rows * ((in_dim + group_size - 1) / group_size);
    check_range(h, s_off, groups * 2, where);
    check_range(h, b_off, groups * 2, where);
    return {at_offset(h, w_off), at_offset(h, s_off), at_offset(h, b_off)};
}

torch::Tensor dequant_affine_q4(const Handle& h, std::vector<int64_t> weight_shape, int64_t weight_offset,
                                int64_t scale_offset, int64_t bias_offset, int group_size,
                                c10::optional<torch::Tensor> output) {
    check_handle(h, "py_dequant_affine_q4");
    if (weight_shape.size() < 2) throw std::runtime_error("py_dequant_affine_q4: weight_shape must have >= 2 dims");
    int64_t n = 1;
    for (auto s : weight_shape) n *= s;
    const int64_t in_dim = weight_shape.back();
    const auto p = affine_ptrs(h, n / std::max<int64_t>(in_dim, 1), in_dim, weight_offset, scale_offset,
                               bias_offset, group_size, "py_dequant_affine_q4");
    torch::Tensor out;
    if (output.has_value()) {
        out = output.value();
        if (out.numel() < n)
            throw std::runtime_error("py_dequant_affine_q4: scratch buffer too small (" +
                                     std::to_string(out.numel()) + " < " + std::to_string(n) + ")");
        if (out.scalar_type() != torch::kFloat16 || !out.is_cuda() || !out.is_contiguous())
            throw std::runtime_error("py_dequant_affine_q4: scratch must be a contiguous float16 GPU tensor");
        out = out.flatten().slice(0, 0, n).view(weight_shape);
    } else {
        out = torch::empty(weight_shape, fp16_on(h->device_id()));
    }
    check(gdsllm_dequant_affine_q4(p.w, p.s, p.b, out.data_ptr(), n, in_dim, group_size, OnDevice(h->device_id()).stream()),
          "py_dequant_affine_q4");
    return out;
}

torch::Tensor fused_affine_q4_gemv(const Handle& h, torch::Tensor x, std::vector<int64_t> weight_shape,
                                   int64_t weight_offset, int64_t scale_offset, int64_t bias_offset, int group_size) {
    check_handle(h, "py_fused_affine_q4_gemv");
    if (weight_shape.size() != 2)
        throw std::runtime_error("py_fused_affine_q4_gemv: weight_shape must be [out_dim, in_dim]");
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    torch::Tensor xf = x.contiguous();
    const int64_t numel = xf.numel();
    int64_t batch = 1;
    if (numel != in_dim) {
        if (in_dim > 0 && numel % in_dim == 0 && numel / in_dim <= 8 && xf.dim() >= 2 && xf.size(-1) == in_dim)
            batch = numel / in_dim;
        else
            throw std::runtime_error("py_fused_affine_q4_gemv: input size " + std::to_string(numel) +
                                     " != in_dim " + std::to_string(in_dim));
    }
    check_x(xf, h->device_id(), "py_fused_affine_q4_gemv");
    const auto p = affine_ptrs(h, out_dim, in_dim, weight_offset, scale_offset, bias_offset, group_size,
                               "py_fused_affine_q4_gemv");
    torch::Tensor out = torch::empty({batch, out_dim}, fp16_on(h->device_id()));
    check(gdsllm_fused_affine_q4_gemv(p.w, p.s, p.b, xf.data_ptr(), out.data_ptr(), out_dim, in_dim, group_size,
                                      batch, in_dim, out_dim, OnDevice(h->device_id()).stream()),
          "py_fused_affine_q4_gemv");
    return out;
}

// ---- extensions beyond the reference module ------------------------------------

// Stacked experts of one projection, described like the layer-file entry
// (runtime/torch_bridge.py:134-145 for a 3-D [E, N, K] affine_q4 tensor).
gdsllm_affine_experts experts_of(const Handle& h, const std::vector<int64_t>& shape, int64_t w_off, int64_t s_off,
                                 int64_t b_off, int64_t group_size, const char* where) {
    check_handle(h, where);
    if (shape.size() != 3) throw std::runtime_error(std::string(where) + ": expert shape must be [E, out_dim, in_dim]");
    const int64_t E = shape[0], N = shape[1], K = shape[2];
    if (group_size <= 0 || K % group_size != 0 || K % 8 != 0)
        throw std::runtime_error(std::string(where) + ": in_dim must be a multiple of 8 and of group_size");
    affine_ptrs(h, E * N, K, w_off, s_off, b_off, group_size, where);
    gdsllm_affine_experts e;
    e.weight = at_offset(h, w_off);
    e.scales = at_offset(h, s_off);
    e.biases = at_offset(h, b_off);
    e.weight_stride = N * (K / 8) * 4;
    e.scale_stride = N * (K / group_size) * 2;
    e.bias_stride = e.scale_stride;
    e.num_experts = E;
    e.out_dim = N;
    e.in_dim = K;
    e.group_size = group_size;
    return e;
}

// Decode top-k expert MLP over resident stacked experts: returns [1, hidden].
torch::Tensor moe_gather_affine_q4(torch::Tensor x, const Handle& gate_h, std::vector<int64_t> gate_shape,
                                   int64_t gate_w, int64_t gate_s, int64_t gate_b, const Handle& up_h,
                                   std::vector<int64_t> up_shape, int64_t up_w, int64_t up_s, int64_t up_b,
                                   const Handle& down_h, std::vector<int64_t> down_shape, int64_t down_w,
                                   int64_t down_s, int64_t down_b, int group_size, torch::Tensor top_k_indices,
                                   torch::Tensor top_k_weights) {
    const char* where = "moe_gather_affine_q4";
    const auto g = experts_of(gate_h, gate_shape, gate_w, gate_s, gate_b, group_size, where);
    const auto u = experts_of(up_h, up_shape, up_w, up_s, up_b, group_size, where);
    const auto d = experts_of(down_h, down_shape, down_w, down_s, down_b, group_size, where);
    const int dev = gate_h->device_id();
    torch::Tensor xf = x.contiguous();
    check_x(xf, dev, where);
    if (xf.numel() != g.in_dim)
        throw std::runtime_error(std::string(where) + ": input size " + std::to_string(xf.numel()) +
                                 " != hidden " + std::to_string(g.in_dim));
    torch::Tensor idx = top_k_indices.reshape({-1}).to(torch::TensorOptions().dtype(torch::kInt32).device(torch::kCUDA, dev)).contiguous();
    torch::Tensor wts = top_k_weights.reshape({-1}).to(torch::TensorOptions().dtype(torch::kFloat16).device(torch::kCUDA, dev)).contiguous();
    const int64_t k = idx.numel();
    if (wts.numel() != k) throw std::runtime_error(std::string(where) + ": indices and weights differ in length");
    const size_t ws_bytes = gdsllm_moe_gather_workspace_size(k, g.out_dim);
    torch::Tensor ws = torch::empty({static_cast<int64_t>(ws_bytes)}, torch::TensorOptions().dtype(torch::kUInt8).device(torch::kCUDA, dev));
    torch::Tensor out = torch::empty({1, d.out_dim}, fp16_on(dev));
    check(gdsllm_moe_gather_affine_q4(&g, &u, &d, xf.data_ptr(), idx.data_ptr<int32_t>(), wts.data_ptr(), k,
                                      out.data_ptr(), ws.data_ptr(), ws_bytes, OnDevice(dev).stream()),
          where);
    return out;
}

// One affine_q4 entry of the layer file: (handle, shape, weight/scale/bias
// offsets, group_size); a 2-D [N, K] shape is one expert.
using AffineEntry = std::tuple<Handle, std::vector<int64_t>, int64_t, int64_t, int64_t, int64_t>;

gdsllm_affine_experts experts_of(const AffineEntry& a, const char* where) {
    std::vector<int64_t> shape = std::get<1>(a);
    if (shape.size() == 2) shape.insert(shape.begin(), 1);
    return experts_of(std::get<0>(a), shape, std::get<2>(a), std::get<3>(a), std::get<4>(a), std::get<5>(a), where);
}

// Decode MoE MLP after routing with the shared expert, its gate and the
// combine fused: entries = (gate, up, down, shared_gate, shared_up,
// shared_down), shared_gate_weight fp16 [1, hidden]; returns [1, hidden] =
// clamp(routed + fp16(sigmoid(g)) * shared), or None for shapes outside the
// fused kernels.
std::optional<torch::Tensor> moe_step_affine_q4(torch::Tensor x, std::vector<AffineEntry> entries,
                                                torch::Tensor top_k_indices, torch::Tensor top_k_weights,
                                                torch::Tensor shared_gate_weight) {
    const char* where = "moe_step_affine_q4";
    if (entries.size() != 6)
        throw std::runtime_error(std::string(where) + ": expects gate, up, down, shared gate, shared up, shared down");
    gdsllm_affine_experts e[6];
    for (int i = 0; i < 6; ++i) e[i] = experts_of(entries[i], where);
    const int dev = std::get<0>(entries[0])->device_id();
    torch::Tensor xf = x.contiguous();
    check_x(xf, dev, where);
    if (xf.numel() != e[0].in_dim)
        throw std::runtime_error(std::string(where) + ": input size " + std::to_string(xf.numel()) +
                                 " != hidden " + std::to_string(e[0].in_dim));
    torch::Tensor sg = shared_gate_weight.contiguous();
    check_x(sg, dev, where);
    if (sg.numel() != e[0].in_dim)
        throw std::runtime_error(std::string(where) + ": shared gate weight must hold hidden values");
    torch::Tensor idx = top_k_indices.reshape({-1}).to(torch::TensorOptions().dtype(torch::kInt32).device(torch::kCUDA, dev)).contiguous();
    torch::Tensor wts = top_k_weights.reshape({-1}).to(torch::TensorOptions().dtype(torch::kFloat16).device(torch::kCUDA, dev)).contiguous();
    const int64_t k = idx.numel();
    if (wts.numel() != k) throw std::runtime_error(std::string(where) + ": indices and weights differ in length");
    const size_t ws_bytes = gdsllm_moe_step_workspace_size(k, e[0].out_dim);
    torch::Tensor ws = torch::empty({static_cast<int64_t>(ws_bytes)}, torch::TensorOptions().dtype(torch::kUInt8).device(torch::kCUDA, dev));
    torch::Tensor out = torch::empty({1, e[2].out_dim}, fp16_on(dev));
    const int rc = gdsllm_moe_step_affine_q4(&e[0], &e[1], &e[2], &e[3], &e[4], &e[5], xf.data_ptr(),
                                             idx.data_ptr<int32_t>(), wts.data_ptr(), k, sg.data_ptr(), out.data_ptr(),
                                             ws.data_ptr(), ws_bytes, OnDevice(dev).stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return std::nullopt;  // the caller runs the separate launches
    check(rc, where);
    return out;
}

// Prefill: x [..., in_dim] fp16 -> [..., out_dim] fp16 on the MFMA dequant-GEMM
// (Q4_0 or Q8_0).  None when the library cannot serve the shape or alignment
// (the caller then takes the reference's dequant -> F.linear route).
std::optional<torch::Tensor> fused_dequant_gemm(const Handle& h, torch::Tensor x, std::vector<int64_t> weight_shape,
                                                const std::string& gguf_type, int64_t offset) {
    const char* where = "fused_dequant_gemm";
    check_handle(h, where);
    if (weight_shape.size() != 2) throw std::runtime_error(std::string(where) + ": weight_shape must be [out_dim, in_dim]");
    if (gguf_type != "q4_0" && gguf_type != "q8_0")
        throw std::runtime_error(std::string(where) + ": unsupported type '" + gguf_type + "'");
    const bool q4 = gguf_type == "q4_0";
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    torch::Tensor xf = x.contiguous();
    check_x(xf, h->device_id(), where);
    if (in_dim <= 0 || xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": last dim of x must equal in_dim " + std::to_string(in_dim));
    const int64_t tokens = xf.numel() / in_dim;
    check_range(h, offset, out_dim * (in_dim / 32) * (q4 ? 18 : 34), where);
    auto out_shape = xf.sizes().vec();
    out_shape.back() = out_dim;
    torch::Tensor out = torch::empty(out_shape, fp16_on(h->device_id()));
    const int rc = (q4 ? gdsllm_dequant_gemm_q4_0 : gdsllm_dequant_gemm_q8_0)(
        at_offset(h, offset), xf.data_ptr(), out.data_ptr(), out_dim, in_dim, tokens, in_dim, out_dim,
        OnDevice(h->device_id()).stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return std::nullopt;
    check(rc, where);
    return out;
}

// Prefill MLP input: h = fp16(fp16(silu(gate x)) * (up x)), x [..., in_dim] ->
// h [..., out_dim] in one MFMA launch over both GGUF matrices (Q4_0 or Q8_0).
// None when the library cannot serve the shape or alignment (the caller then
// runs the two projections and the elementwise SiLU and product).
std::optional<torch::Tensor> fused_gate_up_silu_gemm(const Handle& gate, const Handle& up, torch::Tensor x,
                                                     std::vector<int64_t> weight_shape, const std::string& gguf_type,
                                                     int64_t gate_offset, int64_t up_offset) {
    const char* where = "fused_gate_up_silu_gemm";
    check_handle(gate, where);
    check_handle(up, where);
    if (weight_shape.size() != 2) throw std::runtime_error(std::string(where) + ": weight_shape must be [out_dim, in_dim]");
    if (gguf_type != "q4_0" && gguf_type != "q8_0")
        throw std::runtime_error(std::string(where) + ": unsupported type '" + gguf_type + "'");
    if (gate->device_id() != up->device_id()) throw std::runtime_error(std::string(where) + ": buffers on different devices");
    const bool q4 = gguf_type == "q4_0";
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    torch::Tensor xf = x.contiguous();
    const int dev = gate->device_id();
    check_x(xf, dev, where);
    if (in_dim <= 0 || in_dim % 32 != 0 || xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": last dim of x must equal in_dim " + std::to_string(in_dim) +
                                 " (a multiple of 32)");
    const int64_t tokens = xf.numel() / in_dim;
    check_range(gate, gate_offset, out_dim * (in_dim / 32) * (q4 ? 18 : 34), where);
    check_range(up, up_offset, out_dim * (in_dim / 32) * (q4 ? 18 : 34), where);
    auto out_shape = xf.sizes().vec();
    out_shape.back() = out_dim;
    torch::Tensor h = torch::empty(out_shape, fp16_on(dev));
    const int rc = (q4 ? gdsllm_dequant_gemm_gate_up_silu_q4_0 : gdsllm_dequant_gemm_gate_up_silu_q8_0)(
        at_offset(gate, gate_offset), at_offset(up, up_offset), xf.data_ptr(), h.data_ptr(), out_dim, in_dim, tokens,
        in_dim, out_dim, OnDevice(dev).stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return std::nullopt;
    check(rc, where);
    return h;
}

// Prefill affine-Q4 projection: x [..., in_dim] -> [..., out_dim] on the MFMA
// dequant-GEMM; None for shapes, groupings or alignments it does not serve.
std::optional<torch::Tensor> fused_affine_q4_gemm(const Handle& h, torch::Tensor x, std::vector<int64_t> weight_shape,
                                                  int64_t weight_offset, int64_t scale_offset, int64_t bias_offset,
                                                  int64_t group_size) {
    const char* where = "fused_affine_q4_gemm";
    check_handle(h, where);
    if (weight_shape.size() != 2) throw std::runtime_error(std::string(where) + ": weight_shape must be [out_dim, in_dim]");
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    torch::Tensor xf = x.contiguous();
    check_x(xf, h->device_id(), where);
    if (in_dim <= 0 || xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": last dim of x must equal in_dim " + std::to_string(in_dim));
    const int64_t tokens = xf.numel() / in_dim;
    const auto p = affine_ptrs(h, out_dim, in_dim, weight_offset, scale_offset, bias_offset, group_size, where);
    auto out_shape = xf.sizes().vec();
    out_shape.back() = out_dim;
    torch::Tensor out = torch::empty(out_shape, fp16_on(h->device_id()));
    const int rc = gdsllm_dequant_gemm_affine_q4(p.w, p.s, p.b, xf.data_ptr(), out.data_ptr(), out_dim, in_dim,
                                                 group_size, tokens, in_dim, out_dim, OnDevice(h->device_id()).stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return std::nullopt;
    check(rc, where);
    return out;
}

// Prefill routed-expert MLP over resident stacked experts (the prefill branch
// of runtime/qwen_moe.py:475-492): x [T, hidden], top-k indices / weights
// [T, k]; returns expert_output [T, hidden] fp16, or None for shapes the
// grouped GEMM does not serve.
std::optional<torch::Tensor> moe_prefill_affine_q4(torch::Tensor x, std::vector<AffineEntry> entries,
                                                   torch::Tensor top_k_indices, torch::Tensor top_k_weights) {
    const char* where = "moe_prefill_affine_q4";
    if (entries.size() != 3) throw std::runtime_error(std::string(where) + ": expects gate, up, down");
    gdsllm_affine_experts e[3];
    for (int i = 0; i < 3; ++i) e[i] = experts_of(entries[i], where);
    const int dev = std::get<0>(entries[0])->device_id();
    torch::Tensor xf = x.contiguous();
    check_x(xf, dev, where);
    const int64_t H = e[0].in_dim;
    if (xf.size(-1) != H) throw std::runtime_error(std::string(where) + ": last dim of x must equal hidden " + std::to_string(H));
    const int64_t T = xf.numel() / H;
    torch::Tensor idx = top_k_indices.to(torch::TensorOptions().dtype(torch::kInt32).device(torch::kCUDA, dev)).contiguous();
    torch::Tensor wts = top_k_weights.to(torch::TensorOptions().dtype(torch::kFloat16).device(torch::kCUDA, dev)).contiguous();
    if (T == 0 || idx.numel() % T != 0 || wts.numel() != idx.numel())
        throw std::runtime_error(std::string(where) + ": indices and weights must be [tokens, k]");
    const int64_t k = idx.numel() / T;
    const size_t ws_bytes = gdsllm_moe_prefill_workspace_size(T, k, e[0].out_dim, H, e[0].num_experts);
    torch::Tensor ws = torch::empty({static_cast<int64_t>(ws_bytes)}, torch::TensorOptions().dtype(torch::kUInt8).device(torch::kCUDA, dev));
    torch::Tensor out = torch::empty({T, H}, fp16_on(dev));
    const int rc = gdsllm_moe_prefill_affine_q4(&e[0], &e[1], &e[2], xf.data_ptr(), H, idx.data_ptr<int32_t>(),
                                                wts.data_ptr(), T, k, out.data_ptr(), H, ws.data_ptr(), ws_bytes,
                                                OnDevice(dev).stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return std::nullopt;
    check(rc, where);
    return out;
}

// ---- on-device MoE routing and epilogue (no counterpart op in the reference's
// module: they replace the torch calls of runtime/qwen_moe.py:408-412, 505-513)

void check_fp16_cuda(const torch::Tensor& t, const char* what, const char* where) {
    if (!t.is_cuda() || t.scalar_type() != torch::kFloat16)
        throw std::runtime_error(std::string(where) + ": " + what + " must be a float16 GPU tensor");
}

torch::Tensor gemv_f16(torch::Tensor weight, torch::Tensor x) {
    const char* where = "gemv_f16";
    check_fp16_cuda(weight, "weight", where);
    check_fp16_cuda(x, "x", where);
    if (weight.dim() != 2) throw std::runtime_error(std::string(where) + ": weight must be [out_dim, in_dim]");
    torch::Tensor w = weight.contiguous(), xf = x.contiguous();
    const int64_t out_dim = w.size(0), in_dim = w.size(1);
    if (xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": last dim of x must equal in_dim " + std::to_string(in_dim));
    const int64_t rows = in_dim ? xf.numel() / in_dim : 0;
    auto out_shape = xf.sizes().vec();
    out_shape.back() = out_dim;
    torch::Tensor out = torch::empty(out_shape, w.options());
    const int dev = w.get_device();
    for (int64_t r0 = 0; r0 < rows; r0 += 8) {
        const int64_t nb = std::min<int64_t>(8, rows - r0);
        check(gdsllm_gemv_f16(w.data_ptr(), static_cast<const at::Half*>(xf.data_ptr()) + r0 * in_dim,
                              static_cast<at::Half*>(out.data_ptr()) + r0 * out_dim, out_dim, in_dim, nb, in_dim,
                              out_dim, OnDevice(dev).stream()),
              where);
    }
    return out;
}

// ---- per-column int8 weights (runtime/llama.py:162-165) -------------------------

void check_int8_weights(const torch::Tensor& w, const torch::Tensor& scale, const char* where) {
    if (!w.is_cuda() || w.scalar_type() != torch::kInt8 || w.dim() != 2)
        throw std::runtime_error(std::string(where) + ": weight must be a 2-D int8 CUDA tensor");
    check_fp16_cuda(scale, "scale", where);
    if (scale.numel() != w.size(1))
        throw std::runtime_error(std::string(where) + ": scale must hold one value per input column (" +
                                 std::to_string(w.size(1)) + ")");
    if (scale.get_device() != w.get_device())
        throw std::runtime_error(std::string(where) + ": weight and scale must be on the same device");
}

// (w.float() * scale).half(), bit-exact, into `output` when given.
torch::Tensor dequant_int8(torch::Tensor weight, torch::Tensor scale, c10::optional<torch::Tensor> output) {
    const char* where = "dequant_int8";
    check_int8_weights(weight, scale, where);
    torch::Tensor w = weight.contiguous(), s = scale.contiguous();
    torch::Tensor out;
    if (output.has_value() && output->defined()) {
        out = *output;
        check_fp16_cuda(out, "output", where);
        if (out.numel() < w.numel() || !out.is_contiguous())
            throw std::runtime_error(std::string(where) + ": output must be a contiguous fp16 tensor of " +
                                     std::to_string(w.numel()) + " elements");
        out = out.view(-1).narrow(0, 0, w.numel()).view(w.sizes());
    } else {
        out = torch::empty(w.sizes(), s.options());
    }
    check(gdsllm_dequant_int8(w.data_ptr(), s.data_ptr(), out.data_ptr(), w.size(0), w.size(1),
                              OnDevice(w.get_device()).stream()),
          where);
    return out;
}

// F.linear(x, (w.float() * scale).half()) for x [..., in_dim] fp16: the fused
// GEMV for up to 8 rows of x, else the bit-exact dequant and one GEMM.
torch::Tensor int8_linear(torch::Tensor weight, torch::Tensor scale, torch::Tensor x) {
    const char* where = "int8_linear";
    check_int8_weights(weight, scale, where);
    check_fp16_cuda(x, "x", where);
    if (x.get_device() != weight.get_device())
        throw std::runtime_error(std::string(where) + ": x must be on the weight's device");
    torch::Tensor w = weight.contiguous(), s = scale.contiguous(), xf = x.contiguous();
    const int64_t out_dim = w.size(0), in_dim = w.size(1);
    if (xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": last dim of x must equal in_dim " + std::to_string(in_dim));
    const int64_t rows = in_dim ? xf.numel() / in_dim : 0;
    auto out_shape = xf.sizes().vec();
    out_shape.back() = out_dim;
    if (rows > 8) {
        // bounded fp16 temporaries, as the reference bounds its fp32 ones
        // (runtime/scheduler.py:59-67): row chunks of at most 512 MiB
        const int64_t step = std::max<int64_t>(1, (int64_t(512) << 20) / std::max<int64_t>(1, 2 * in_dim));
        if (out_dim <= step) return at::linear(xf, dequant_int8(w, s, c10::nullopt)).view(out_shape);
        std::vector<torch::Tensor> parts;
        for (int64_t r = 0; r < out_dim; r += step)
            parts.push_back(at::linear(xf, dequant_int8(w.narrow(0, r, std::min(step, out_dim - r)), s, c10::nullopt)));
        return at::cat(parts, -1).view(out_shape);
    }
    torch::Tensor out = torch::empty(out_shape, xf.options());
    if (rows == 0) return out;
    check(gdsllm_fused_int8_gemv(w.data_ptr(), s.data_ptr(), xf.data_ptr(), out.data_ptr(), out_dim, in_dim, rows,
                                 in_dim, out_dim, OnDevice(w.get_device()).stream()),
          where);
    return out;
}

py::tuple moe_route_topk(torch::Tensor logits, int64_t top_k) {
    const char* where = "moe_route_topk";
    check_fp16_cuda(logits, "logits", where);
    torch::Tensor l = logits.contiguous();
    const int64_t E = l.size(-1), n = E ? l.numel() / E : 0;
    auto shape = l.sizes().vec();
    shape.back() = top_k;
    torch::Tensor idx = torch::empty(shape, l.options().dtype(torch::kInt32));
    torch::Tensor w = torch::empty(shape, l.options());
    check(gdsllm_moe_route_topk(l.data_ptr(), E, n, E, top_k, idx.data_ptr<int32_t>(), w.data_ptr(),
                                OnDevice(l.get_device()).stream()),
          where);
    return py::make_tuple(idx, w);
}

torch::Tensor moe_combine(torch::Tensor expert_out, torch::Tensor shared_out, torch::Tensor shared_gate_logit) {
    const char* where = "moe_combine";
    check_fp16_cuda(expert_out, "expert_out", where);
    check_fp16_cuda(shared_out, "shared_out", where);
    check_fp16_cuda(shared_gate_logit, "shared_gate_logit", where);
    torch::Tensor e = expert_out.contiguous(), s = shared_out.contiguous(), g = shared_gate_logit.contiguous();
    if (!e.sizes().equals(s.sizes())) throw std::runtime_error(std::string(where) + ": expert_out and shared_out differ in shape");
    const int64_t H = e.size(-1), n = H ? e.numel() / H : 0;
    if (g.numel() != n) throw std::runtime_error(std::string(where) + ": one gate logit per row expected");
    torch::Tensor y = torch::empty_like(e);
    check(gdsllm_moe_combine(e.data_ptr(), s.data_ptr(), g.data_ptr(), y.data_ptr(), H, n, OnDevice(e.get_device()).stream()),
          where);
    return y;
}

// q/k/v-style projections sharing x in one launch (the decode step's
// runtime/llama.py:212-214): one output [batch, out_dim_i] per matrix.
std::vector<torch::Tensor> fused_dequant_gemv_group(const std::vector<Handle>& handles, torch::Tensor x,
                                                    const std::vector<std::vector<int64_t>>& weight_shapes,
                                                    const std::string& gguf_type,
                                                    const std::vector<int64_t>& offsets) {
    const char* where = "py_fused_dequant_gemv_group";
    const size_t n = handles.size();
    if (n < 1 || n > 4 || weight_shapes.size() != n || offsets.size() != n)
        throw std::runtime_error(std::string(where) + ": 1 to 4 handles with one shape and offset each");
    const int64_t bb = gguf_block_bytes(gguf_type, where);
    const int64_t in_dim = weight_shapes[0].size() == 2 ? weight_shapes[0][1] : -1;
    for (size_t i = 0; i < n; ++i) {
        check_handle(handles[i], where);
        if (weight_shapes[i].size() != 2 || weight_shapes[i][1] != in_dim)
            throw std::runtime_error(std::string(where) + ": weight shapes must be [out_dim, in_dim] with one in_dim");
        if (handles[i]->device_id() != handles[0]->device_id())
            throw std::runtime_error(std::string(where) + ": buffers on different devices");
        check_range(handles[i], offsets[i], weight_shapes[i][0] * (in_dim / 32) * bb, where);
    }
    if (in_dim % 32 != 0) throw std::runtime_error(std::string(where) + ": in_dim must be a multiple of 32");
    torch::Tensor xf = x.contiguous();
    const int64_t batch = in_dim > 0 ? xf.numel() / in_dim : 0;
    if (batch < 1 || batch > 8 || batch * in_dim != xf.numel() || xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": x must be [batch <= 8, in_dim]");
    const int dev = handles[0]->device_id();
    check_x(xf, dev, where);
    std::vector<torch::Tensor> outs;
    const void* w[4];
    void* y[4];
    int64_t m[4];
    for (size_t i = 0; i < n; ++i) {
        outs.push_back(torch::empty({batch, weight_shapes[i][0]}, fp16_on(dev)));
        w[i] = at_offset(handles[i], offsets[i]);
        y[i] = outs.back().data_ptr();
        m[i] = weight_shapes[i][0];
    }
    const OnDevice on(dev);
    const int rc = gguf_type == "q4_0"
                       ? gdsllm_fused_q4_0_gemv_group(static_cast<int>(n), w, y, m, xf.data_ptr(), in_dim, batch,
                                                      in_dim, on.stream())
                       : gdsllm_fused_q8_0_gemv_group(static_cast<int>(n), w, y, m, xf.data_ptr(), in_dim, batch,
                                                      in_dim, on.stream());
    check(rc, where);
    return outs;
}

// h = fp16(silu(fp16(gate . x)) * fp16(up . x)) in one launch (the MLP's
// runtime/llama.py:253-256 before the down projection).  Returns None when
// the shape is outside the fused kernel (batch > 2, in_dim % 256 != 0): the
// caller then runs the projections separately.
py::object fused_gate_up_silu(const Handle& gate, const Handle& up, torch::Tensor x,
                              std::vector<int64_t> weight_shape, const std::string& gguf_type, int64_t gate_offset,
                              int64_t up_offset) {
    const char* where = "py_fused_gate_up_silu";
    check_handle(gate, where);
    check_handle(up, where);
    if (weight_shape.size() != 2) throw std::runtime_error(std::string(where) + ": weight_shape must be [out_dim, in_dim]");
    const int64_t out_dim = weight_shape[0], in_dim = weight_shape[1];
    if (in_dim % 32 != 0) throw std::runtime_error(std::string(where) + ": in_dim must be a multiple of 32");
    const int64_t bb = gguf_block_bytes(gguf_type, where);
    check_range(gate, gate_offset, out_dim * (in_dim / 32) * bb, where);
    check_range(up, up_offset, out_dim * (in_dim / 32) * bb, where);
    if (gate->device_id() != up->device_id()) throw std::runtime_error(std::string(where) + ": buffers on different devices");
    torch::Tensor xf = x.contiguous();
    const int64_t batch = in_dim > 0 ? xf.numel() / in_dim : 0;
    if (batch < 1 || batch * in_dim != xf.numel() || xf.size(-1) != in_dim)
        throw std::runtime_error(std::string(where) + ": x must be [batch, in_dim]");
    const int dev = gate->device_id();
    check_x(xf, dev, where);
    torch::Tensor h = torch::empty({batch, out_dim}, fp16_on(dev));
    const OnDevice on(dev);
    const int rc = gguf_type == "q4_0"
                       ? gdsllm_fused_q4_0_gate_up_silu(at_offset(gate, gate_offset), at_offset(up, up_offset),
                                                        xf.data_ptr(), h.data_ptr(), out_dim, in_dim, batch, in_dim,
                                                        out_dim, on.stream())
                       : gdsllm_fused_q8_0_gate_up_silu(at_offset(gate, gate_offset), at_offset(up, up_offset),
                                                        xf.data_ptr(), h.data_ptr(), out_dim, in_dim, batch, in_dim,
                                                        out_dim, on.stream());
    if (rc == GDSLLM_ERR_UNSUPPORTED) return py::none();
    check(rc, where);
    return py::cast(h);
}

Handle from_tensor(const torch::Tensor& t) { return std::make_shared<GdsBufferHandle>(t); }

}  // namespace

PYBIND11_MODULE(gds_io_ext, m) {
    m.doc() = "gdsllm_amd: HBM-resident weight buffers and MI355X quantized matvec ops";

    m.def("init", &init, "Check that a HIP device is present. Call once at startup.");
    m.def("shutdown", &shutdown, "Counterpart of init().");
    m.def("is_driver_open", &is_driver_open, "True after a successful init().");

    py::class_<GdsBufferHandle, Handle>(m, "GdsBufferHandle", "Handle to an HBM-resident device buffer.")
        .def_property_readonly("size", &GdsBufferHandle::size)
        .def_property_readonly("device_id", &GdsBufferHandle::device_id)
        .def_property_readonly("registered", &GdsBufferHandle::registered)
        .def_property_readonly("data_ptr", &GdsBufferHandle::data_ptr)
        .def_static("from_tensor", &from_tensor, "Wrap (and keep alive) a contiguous GPU tensor's storage.",
                    py::arg("tensor"));

    m.def("load_file", &load_file, "Load an entire file into a device buffer.", py::arg("filepath"),
          py::arg("size_bytes"), py::arg("device_id") = 0);
    m.def("load_file_region", &load_file_region, "Load a contiguous region of a file into a device buffer.",
          py::arg("filepath"), py::arg("size_bytes"), py::arg("file_offset"), py::arg("device_id") = 0);
    m.def("load_expert", &load_expert, "Load one expert's weight+scale+bias into a single device buffer.",
          py::arg("filepath"), py::arg("w_file_offset"), py::arg("w_size"), py::arg("s_file_offset"),
          py::arg("s_size"), py::arg("b_file_offset"), py::arg("b_size"), py::arg("device_id") = 0);
    m.def("view_tensor", &view_tensor, "Create a torch.Tensor view into a buffer at an offset.", py::arg("handle"),
          py::arg("shape"), py::arg("dtype"), py::arg("offset"));
    m.def("load_tensor", &load_tensor, "Load a region of a file directly into a GPU tensor.", py::arg("filepath"),
          py::arg("shape"), py::arg("dtype") = "float16", py::arg("file_offset") = 0, py::arg("size_bytes") = 0,
          py::arg("device_id") = 0);

    m.def("dequant_gguf", &dequant_gguf, "Dequantize GGUF Q4_0/Q8_0 blocks from a buffer to fp16.",
          py::arg("handle"), py::arg("shape"), py::arg("gguf_type"), py::arg("offset"),
          py::arg("output") = py::none());
    m.def("embed_gguf", &embed_gguf, "Embedding rows of a GGUF Q4_0/Q8_0 table, dequantized on the fly.",
          py::arg("handle"), py::arg("token_ids"), py::arg("shape"), py::arg("gguf_type"), py::arg("offset") = 0);
    m.def("fused_dequant_gemv", &fused_dequant_gemv, "Fused dequant + GEMV for Q4_0/Q8_0 (decode).",
          py::arg("handle"), py::arg("x"), py::arg("weight_shape"), py::arg("gguf_type"), py::arg("offset"));
    m.def("fused_dequant_gemv_group", &fused_dequant_gemv_group,
          "Up to 4 fused dequant + GEMVs sharing x in one launch (decode q/k/v).", py::arg("handles"), py::arg("x"),
          py::arg("weight_shapes"), py::arg("gguf_type"), py::arg("offsets"));
    m.def("fused_gate_up_silu", &fused_gate_up_silu,
          "fp16(silu(gate . x) * (up . x)) in one launch (decode MLP); None when the shape needs separate launches.",
          py::arg("gate_handle"), py::arg("up_handle"), py::arg("x"), py::arg("weight_shape"), py::arg("gguf_type"),
          py::arg("gate_offset"), py::arg("up_offset"));
    m.def("dequant_affine_q4", &dequant_affine_q4, "Dequantize affine Q4 (uint32 + scales + biases) to fp16.",
          py::arg("handle"), py::arg("weight_shape"), py::arg("weight_offset"), py::arg("scale_offset"),
          py::arg("bias_offset"), py::arg("group_size"), py::arg("output") = py::none());
    m.def("fused_affine_q4_gemv", &fused_affine_q4_gemv, "Fused affine Q4 dequant + GEMV (decode).",
          py::arg("handle"), py::arg("x"), py::arg("weight_shape"), py::arg("weight_offset"),
          py::arg("scale_offset"), py::arg("bias_offset"), py::arg("group_size"));

    m.def("moe_gather_affine_q4", &moe_gather_affine_q4,
          "Decode top-k expert MLP (gate, up, silu*up, down, weighted sum) over resident stacked experts.",
          py::arg("x"), py::arg("gate_handle"), py::arg("gate_shape"), py::arg("gate_weight_offset"),
          py::arg("gate_scale_offset"), py::arg("gate_bias_offset"), py::arg("up_handle"), py::arg("up_shape"),
          py::arg("up_weight_offset"), py::arg("up_scale_offset"), py::arg("up_bias_offset"),
          py::arg("down_handle"), py::arg("down_shape"), py::arg("down_weight_offset"),
          py::arg("down_scale_offset"), py::arg("down_bias_offset"), py::arg("group_size"),
          py::arg("top_k_indices"), py::arg("top_k_weights"));
    m.def("moe_step_affine_q4", &moe_step_affine_q4,
          "Decode MoE MLP after routing (top-k experts, shared expert, sigmoid-gated combine) in two launches.",
          py::arg("x"), py::arg("entries"), py::arg("top_k_indices"), py::arg("top_k_weights"),
          py::arg("shared_gate_weight"));
    m.def("fused_affine_q4_gemm", &fused_affine_q4_gemm,
          "Prefill affine-Q4 dequant-GEMM on MFMA: x [..., K] -> [..., M] (None if not served).", py::arg("handle"),
          py::arg("x"), py::arg("weight_shape"), py::arg("weight_offset"), py::arg("scale_offset"),
          py::arg("bias_offset"), py::arg("group_size"));
    m.def("moe_prefill_affine_q4", &moe_prefill_affine_q4,
          "Prefill routed-expert MLP over stacked experts: x [T, H] -> expert_output [T, H] (None if not served).",
          py::arg("x"), py::arg("entries"), py::arg("top_k_indices"), py::arg("top_k_weights"));
    m.def("fused_gate_up_silu_gemm", &fused_gate_up_silu_gemm,
          "Prefill fp16(silu(gate . x) * (up . x)) on MFMA: x [..., K] -> h [..., M] (None if not served).",
          py::arg("gate_handle"), py::arg("up_handle"), py::arg("x"), py::arg("weight_shape"), py::arg("gguf_type"),
          py::arg("gate_offset"), py::arg("up_offset"));
    m.def("fused_dequant_gemm", &fused_dequant_gemm, "Prefill Q4_0/Q8_0 dequant-GEMM on MFMA: x [T, K] -> [T, M] (None if not served).",
          py::arg("handle"), py::arg("x"), py::arg("weight_shape"), py::arg("gguf_type"), py::arg("offset"));
    m.def("gemv_f16", &gemv_f16, "fp16-weight GEMV (router, shared-expert gate): x [..., K] -> [..., M].",
          py::arg("weight"), py::arg("x"));
    m.def("dequant_int8", &dequant_int8, "(w.float() * scale).half() of per-column int8 weights, bit-exact.",
          py::arg("weight"), py::arg("scale"), py::arg("output") = py::none());
    m.def("int8_linear", &int8_linear, "F.linear(x, (w.float() * scale).half()) without the fp32 round trip.",
          py::arg("weight"), py::arg("scale"), py::arg("x"));
    m.def("moe_route_topk", &moe_route_topk, "Top-k experts and fp16(softmax_fp32) weights from fp16 logits.",
          py::arg("logits"), py::arg("top_k"));
    m.def("moe_combine", &moe_combine, "clamp(expert_out + sigmoid(gate) * shared_out) with torch fp16 semantics.",
          py::arg("expert_out"), py::arg("shared_out"), py::arg("shared_gate_logit"));
}
