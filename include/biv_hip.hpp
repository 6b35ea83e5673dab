// biv_hip.hpp — C++ host mirror of biv's MoE-block interface over the C ABI
// of biv_hip.h (header only).
//
// biv is Rust; its MoE block is reached through these types and calls
// (engine/src/model.rs, engine/src/engine.rs):
//   Weight::new(ty, cols, rows, data)           ops.rs:22-33        -> Engine::weight
//   Experts { ty, cols, rows, n, data, stride, offset }
//                                               model.rs:190-216    -> Experts, Engine::experts
//   SharedExpert { gate, up, down, gate_inp }   model.rs:218-227    -> SharedExpert
//   Moe { router, gate, up, down, shared }      model.rs:229-237    -> Moe, Engine::moe
//   Model::ffn(layer, h, n) -> Vec<f32>         model.rs:853-898    -> DeviceMoe::ffn
//   Ffn::Dense { gate, up, down }, dense_ffn    model.rs:239-246, 1118-1126 -> DeviceDense::ffn
//   encode_moe (x += moe(h) in device buffers)  metal/mod.rs:2138-2148 -> DeviceMoe::encode
//   Engine::description / device_memory / numerics  engine.rs:15-60
//   Error::Backend(String)                      error.rs:67-68      -> Error
// The names and argument meanings follow those; a failure of the library
// throws Error carrying its BIV_HIP_E_* code and message, where the Rust
// backend returns Error::Backend (construction) or panics (passes), as biv's
// Metal backend does.
//
// Ownership: an Engine owns the device context and every upload and layer
// made through it (freed when the Engine is destroyed); the Weight, Experts
// handles and DeviceMoe / DeviceDense objects it returns are valid while it
// lives.  An Engine is used by one thread at a time.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "biv_hip.h"

namespace biv::hip {

// ggml tensor types of the MoE path (GgmlType, quant.rs:31-48)
enum class GgmlType : int {
    F32 = BIV_GGML_F32,
    F16 = BIV_GGML_F16,
    Q8_0 = BIV_GGML_Q8_0,
    Q4_K = BIV_GGML_Q4_K,
    Q6_K = BIV_GGML_Q6_K,
    BF16 = BIV_GGML_BF16,
};

// Bytes of a row of n elements (GgmlType::row_size)
inline size_t row_size(GgmlType ty, size_t n)
{
    switch (ty) {
    case GgmlType::F32: return 4 * n;
    case GgmlType::F16:
    case GgmlType::BF16: return 2 * n;
    case GgmlType::Q8_0: return n / 32 * 34;
    case GgmlType::Q4_K: return n / 256 * 144;
    case GgmlType::Q6_K: return n / 256 * 210;
    }
    return 0;
}

// Error::Backend(String), with the library's code
class Error : public std::runtime_error {
  public:
    Error(int code, const std::string &msg) : std::runtime_error(msg), code_(code) {}
    int code() const { return code_; }

  private:
    int code_;
};

// A stack of matrices of one shape in host memory, one per expert (Experts)
struct Experts {
    GgmlType ty;
    size_t cols, rows, n;
    const void *data;
    size_t stride; // bytes from an expert's matrix to the next
    size_t offset; // bytes from an expert's matrix to these rows (the up half of a fused gate/up)
};

// Host descriptions of the parts of a MoE block and a dense FFN
struct HostWeight {
    GgmlType ty;
    size_t cols, rows;
    const void *data;
};
struct SharedExpert {
    HostWeight gate, up, down, gate_inp;
};
struct Moe {
    HostWeight router;
    Experts gate, up, down;
    const SharedExpert *shared; // nullptr: no shared expert
    int k;                      // n_expert_used
};

class Engine;

// Model::ffn / encode_moe for one MoE layer on the device
class DeviceMoe {
  public:
    size_t n_embd() const { return n_embd_; }
    // Model::ffn (model.rs:853-898): moe(h) of n rows of h [n x n_embd], host memory
    std::vector<float> ffn(const float *h, size_t n) const;
    // the residual form, x += moe(h) (model.rs:788-790), host memory
    void ffn_add(const float *h, size_t n, float *x) const;
    // encode_moe: x (+)= moe(h) with device pointers, queued on the engine's stream
    void encode(const float *h_dev, size_t n, float *x_dev, bool add) const;
    // the FFN half of Model::layer in device memory: x += moe(rms_norm(x))
    void ffn_step(float *x_dev, const float *norm_dev, float eps, size_t n) const;
    const biv_hip_moe *raw() const { return moe_; }

  private:
    friend class Engine;
    DeviceMoe(biv_hip_ctx *ctx, biv_hip_moe *moe, size_t n_embd) : ctx_(ctx), moe_(moe), n_embd_(n_embd) {}
    biv_hip_ctx *ctx_;
    biv_hip_moe *moe_;
    size_t n_embd_;
};

// Model::ffn for a dense layer (Ffn::Dense, dense_ffn)
class DeviceDense {
  public:
    size_t n_embd() const { return n_embd_; }
    std::vector<float> ffn(const float *h, size_t n) const;

  private:
    friend class Engine;
    DeviceDense(biv_hip_ctx *ctx, biv_hip_dense *d, size_t n_embd) : ctx_(ctx), d_(d), n_embd_(n_embd) {}
    biv_hip_ctx *ctx_;
    biv_hip_dense *d_;
    size_t n_embd_;
};

// The device context: the backend part of biv's Engine for the FFN blocks
class Engine {
  public:
    explicit Engine(int device = 0)
    {
        if (int rc = biv_hip_create(device, &ctx_)) throw Error(rc, biv_hip_last_error(nullptr));
    }
    ~Engine() { biv_hip_destroy(ctx_); }
    Engine(const Engine &) = delete;
    Engine &operator=(const Engine &) = delete;
    Engine(Engine &&o) noexcept : ctx_(std::exchange(o.ctx_, nullptr)) {}

    // Engine::description
    std::string description() const
    {
        return "biv hip backend (gfx950): MoE and dense FFN blocks, " + std::to_string(device_memory() >> 20) +
               " MiB uploaded";
    }
    // bytes of device memory held by the uploads (Engine::device_memory's allocated part)
    size_t device_memory() const { return biv_hip_device_bytes(ctx_); }
    // Engine::numerics: (name, value) pairs
    std::vector<std::pair<std::string, std::string>> numerics() const
    {
        char buf[1024];
        check(biv_hip_numerics(ctx_, buf, sizeof buf));
        std::vector<std::pair<std::string, std::string>> out;
        std::string s(buf);
        size_t i = 0;
        while (i < s.size()) {
            size_t j = s.find(';', i);
            if (j == std::string::npos) j = s.size();
            const std::string kv = s.substr(i, j - i);
            const size_t eq = kv.find('=');
            if (!kv.empty()) out.emplace_back(kv.substr(0, eq), eq == std::string::npos ? "" : kv.substr(eq + 1));
            i = j + 1;
        }
        return out;
    }
    void sync() const { check(biv_hip_sync(ctx_)); }

    // Weight::new: one matrix copied to the device
    const biv_hip_weight *weight(const HostWeight &w) const
    {
        biv_hip_weight *out = nullptr;
        check(biv_hip_upload_weight(ctx_, static_cast<int>(w.ty), w.cols, w.rows, w.data, &out));
        return out;
    }
    // Experts: a stack copied to the device
    const biv_hip_experts *experts(const Experts &x) const
    {
        biv_hip_experts *out = nullptr;
        check(biv_hip_upload_experts(ctx_, static_cast<int>(x.ty), x.cols, x.rows, x.n, x.data, x.stride,
                                     x.offset, &out));
        return out;
    }
    // struct Moe on the device: uploads its parts and makes the block
    DeviceMoe moe(const Moe &m) const
    {
        const biv_hip_weight *router = weight(m.router);
        const biv_hip_experts *g = experts(m.gate), *u = experts(m.up), *d = experts(m.down);
        const biv_hip_weight *sg = nullptr, *su = nullptr, *sd = nullptr, *gi = nullptr;
        if (m.shared) {
            sg = weight(m.shared->gate);
            su = weight(m.shared->up);
            sd = weight(m.shared->down);
            gi = weight(m.shared->gate_inp);
        }
        biv_hip_moe *out = nullptr;
        check(biv_hip_moe_create(ctx_, router, g, u, d, sg, su, sd, gi, m.k, &out));
        return DeviceMoe(ctx_, out, m.router.cols);
    }
    // Ffn::Dense on the device
    DeviceDense dense(const HostWeight &gate, const HostWeight &up, const HostWeight &down) const
    {
        const biv_hip_weight *g = weight(gate), *u = weight(up), *d = weight(down);
        biv_hip_dense *out = nullptr;
        check(biv_hip_dense_create(ctx_, g, u, d, &out));
        return DeviceDense(ctx_, out, gate.cols);
    }

    // device buffers for callers without another allocator
    void *malloc(size_t bytes) const
    {
        void *p = nullptr;
        check(biv_hip_malloc(ctx_, bytes, &p));
        return p;
    }
    void free(void *p) const { check(biv_hip_free(ctx_, p)); }
    void h2d(void *dst, const void *src, size_t bytes) const { check(biv_hip_memcpy_h2d(ctx_, dst, src, bytes)); }
    void d2h(void *dst, const void *src, size_t bytes) const { check(biv_hip_memcpy_d2h(ctx_, dst, src, bytes)); }

    biv_hip_ctx *raw() const { return ctx_; }

    // throw Error for a failed call on this context
    void check(int rc) const
    {
        if (rc) throw Error(rc, biv_hip_last_error(ctx_));
    }

  private:
    biv_hip_ctx *ctx_ = nullptr;
};

inline std::vector<float> DeviceMoe::ffn(const float *h, size_t n) const
{
    std::vector<float> out(n * n_embd_);
    if (int rc = biv_hip_moe_forward(ctx_, moe_, h, static_cast<int>(n), out.data(), 0))
        throw Error(rc, biv_hip_last_error(ctx_));
    return out;
}

inline void DeviceMoe::ffn_add(const float *h, size_t n, float *x) const
{
    if (int rc = biv_hip_moe_forward(ctx_, moe_, h, static_cast<int>(n), x, BIV_HIP_ADD))
        throw Error(rc, biv_hip_last_error(ctx_));
}

inline void DeviceMoe::encode(const float *h_dev, size_t n, float *x_dev, bool add) const
{
    if (int rc = biv_hip_moe_forward_device(ctx_, moe_, h_dev, static_cast<int>(n), x_dev, add ? BIV_HIP_ADD : 0))
        throw Error(rc, biv_hip_last_error(ctx_));
}

inline void DeviceMoe::ffn_step(float *x_dev, const float *norm_dev, float eps, size_t n) const
{
    if (int rc = biv_hip_moe_ffn_step(ctx_, moe_, x_dev, norm_dev, eps, static_cast<int>(n)))
        throw Error(rc, biv_hip_last_error(ctx_));
}

inline std::vector<float> DeviceDense::ffn(const float *h, size_t n) const
{
    std::vector<float> out(n * n_embd_);
    if (int rc = biv_hip_dense_forward(ctx_, d_, h, static_cast<int>(n), out.data(), 0))
        throw Error(rc, biv_hip_last_error(ctx_));
    return out;
}

} // namespace biv::hip
