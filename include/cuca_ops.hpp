// cuca_ops.hpp -- C++ host side over the C ABI of cuca_hip.h, mirroring the
// reference engine's per-layer op surface (paths under
// src/provider/local/model/ of nassor/cuca 0.10.0):
//
//   cuca::TokenEmbedding{dtype, data, rows, row_len}.rows(tokens, scale)   quant.rs:352-411
//   cuca::rms(x, weight, eps)                                              cpu.rs:3652
//   cuca::add_rms(x, branch, weight, eps, ...)                             cpu.rs:2650-2711
//   cuca::Glu{act, clamp}.apply(gate, up)                                  cpu.rs:342-371
//   cuca::apply_rope(x, cos, sin, kind, n_dims, positions)                 cpu.rs:3672-3688
//   cuca::RopeSpec::plain(kind, n_dims, base).tables(factors, positions)   rope.rs:62-151
//   cuca::KvPool{n_blocks, n_kv_head, head_dim}.store_kv(q, k, v, ...)     cpu.rs:3028-3097,
//                                                                          gpu.rs:1774-1806
//   cuca::KvPool::decode(q, tables, ranges, n_head, scale)                 paged_kernel.rs:92-282
//
// Tensors are cuca::Tensor: a device buffer owned through the context, with
// a row-major shape and an element type (f32, or f16 held as uint16_t bits).
// Errors are thrown as cuca::Error carrying the library's status and
// message -- the reference's CucaError::Provider(Local, msg)
// (model/mod.rs:222-228).  Header-only; link libcuca_hip.so.
#pragma once

#include "cuca_hip.h"

#include <cstdint>
#include <cstring>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace cuca {

struct Error : std::runtime_error {
    cuca_status status;
    Error(cuca_status st, const std::string &msg) : std::runtime_error(msg), status(st) {}
};

inline void check(const cuca_hip_ctx *ctx, cuca_status st) {
    if (st != CUCA_OK) throw Error(st, cuca_hip_last_error(ctx));
}

// Act (arch.rs:101-106) and RopeKind (rope.rs:28-36).
enum class Act { Silu = CUCA_ACT_SILU, Gelu = CUCA_ACT_GELU_TANH };
enum class RopeKind { Norm = CUCA_ROPE_NORM, Neox = CUCA_ROPE_NEOX };
// Element types: the activation types of cuca_dtype, then the byte, id and
// position buffers the ops also take.
enum class DType { F32 = CUCA_F32, F16 = CUCA_F16, U8 = 100, U32 = 101, I32 = 102 };

inline size_t dtype_size(DType t) {
    switch (t) {
    case DType::F16: return 2;
    case DType::U8: return 1;
    default: return 4;
    }
}

class Context;

// A device buffer with a shape and an element type.  Move-only; freed with
// the context that allocated it.
class Tensor {
  public:
    Tensor() = default;
    Tensor(Context &ctx, std::vector<int64_t> shape, DType dtype);
    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;
    Tensor(Tensor &&o) noexcept { *this = std::move(o); }
    Tensor &operator=(Tensor &&o) noexcept;
    ~Tensor();

    void *data() const { return ptr_; }
    DType dtype() const { return dtype_; }
    const std::vector<int64_t> &shape() const { return shape_; }
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape_) n *= d;
        return n;
    }
    int64_t dim(int i) const { return shape_.at(i < 0 ? shape_.size() + i : i); }
    size_t bytes() const { return (size_t)numel() * dtype_size(dtype_); }

    // Host <-> device (synchronous on the context's stream).
    template <typename E> void upload(const std::vector<E> &host);
    template <typename E> std::vector<E> download() const;

  private:
    Context *ctx_ = nullptr;
    void *ptr_ = nullptr;
    std::vector<int64_t> shape_;
    DType dtype_ = DType::F32;
};

// One cuca_hip context: a gfx950 device, its stream, the loaded kernels.
class Context {
  public:
    explicit Context(int device = 0) {
        cuca_status st = cuca_hip_ctx_create(device, &ctx_);
        if (st != CUCA_OK) throw Error(st, cuca_hip_last_error(nullptr));
    }
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;
    ~Context() { cuca_hip_ctx_destroy(ctx_); }

    cuca_hip_ctx *raw() const { return ctx_; }
    void check(cuca_status st) const { cuca::check(ctx_, st); }
    void sync() const { check(cuca_hip_stream_sync(ctx_)); }
    void check_device() const { check(cuca_hip_check_device(ctx_)); }

    template <typename E>
    Tensor tensor(const std::vector<E> &host, std::vector<int64_t> shape, DType dtype) {
        Tensor t(*this, std::move(shape), dtype);
        t.upload(host);
        return t;
    }

  private:
    cuca_hip_ctx *ctx_ = nullptr;
};

inline Tensor::Tensor(Context &ctx, std::vector<int64_t> shape, DType dtype)
    : ctx_(&ctx), shape_(std::move(shape)), dtype_(dtype) {
    ctx.check(cuca_hip_malloc(ctx.raw(), bytes(), &ptr_));
}

inline Tensor &Tensor::operator=(Tensor &&o) noexcept {
    if (this != &o) {
        if (ctx_ && ptr_) (void)cuca_hip_free(ctx_->raw(), ptr_);
        ctx_ = o.ctx_;
        ptr_ = o.ptr_;
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        o.ptr_ = nullptr;
        o.ctx_ = nullptr;
    }
    return *this;
}

inline Tensor::~Tensor() {
    if (ctx_ && ptr_) (void)cuca_hip_free(ctx_->raw(), ptr_);
}

template <typename E> void Tensor::upload(const std::vector<E> &host) {
    if (host.size() * sizeof(E) != bytes()) throw Error(CUCA_INVALID_ARG, "upload size mismatch");
    ctx_->check(cuca_hip_memcpy_h2d_async(ctx_->raw(), ptr_, host.data(), bytes()));
    ctx_->sync();
}

template <typename E> std::vector<E> Tensor::download() const {
    if (bytes() % sizeof(E) != 0) throw Error(CUCA_INVALID_ARG, "download element size");
    std::vector<E> host(bytes() / sizeof(E));
    ctx_->check(cuca_hip_memcpy_d2h_async(ctx_->raw(), host.data(), ptr_, bytes()));
    ctx_->sync();
    return host;
}

// --------------------------------------------------------------------
// TokenEmbedding (quant.rs:352-411)
// --------------------------------------------------------------------

class TokenEmbedding {
  public:
    // The [rows, row_len] table of ggml type `dtype` (CUCA_GGML_Q4_0 /
    // CUCA_GGML_Q8_0) over its file bytes, uploaded once.
    TokenEmbedding(Context &ctx, uint32_t dtype, const std::vector<uint8_t> &data, int64_t rows,
                   int64_t row_len)
        : ctx_(&ctx), dtype_(dtype), rows_(rows), row_len_(row_len) {
        const char *name = dtype == CUCA_GGML_Q4_0 ? "Q4_0" : dtype == CUCA_GGML_Q8_0 ? "Q8_0" : nullptr;
        if (!name) throw Error(CUCA_UNSUPPORTED, "ggml type " + std::to_string(dtype) +
                                                     ": only Q4_0 and Q8_0 are supported");
        if (row_len % 32 != 0)  // quant.rs:362-367
            throw Error(CUCA_INVALID_ARG, "token embedding: row length " + std::to_string(row_len) +
                                              " is not a whole number of " + name + " blocks");
        const int64_t row_bytes = row_len / 32 * (dtype == CUCA_GGML_Q4_0 ? 18 : 34);
        if (rows * row_bytes != (int64_t)data.size())  // quant.rs:368-374
            throw Error(CUCA_INVALID_ARG, "token embedding: " + std::to_string(data.size()) +
                                              " bytes do not hold " + std::to_string(rows) + " rows of " +
                                              std::to_string(row_len) + " " + name + " values");
        table_ = ctx.tensor(data, {(int64_t)data.size()}, DType::U8);
    }

    // Embedding rows of `tokens`, concatenated and multiplied by `scale`
    // (quant.rs:391-411): a [tokens.size(), row_len] tensor of `out`.
    Tensor rows(const std::vector<uint32_t> &tokens, float scale, DType out = DType::F32) const {
        for (uint32_t id : tokens)  // quant.rs:395-400, before anything runs
            if ((int64_t)id >= rows_)
                throw Error(CUCA_OUT_OF_RANGE, "token id " + std::to_string(id) +
                                                   " outside the embedding table of " +
                                                   std::to_string(rows_) + " rows");
        Tensor result(*ctx_, {(int64_t)tokens.size(), row_len_}, out);
        if (tokens.empty()) return result;
        Tensor ids = ctx_->tensor(tokens, {(int64_t)tokens.size()}, DType::U32);
        ctx_->check(cuca_hip_embed_gguf(ctx_->raw(), table_.data(), dtype_, rows_, row_len_,
                                        static_cast<const uint32_t *>(ids.data()), (int64_t)tokens.size(),
                                        scale, result.data(), (cuca_dtype)out));
        ctx_->sync();  // `ids` is freed on return
        return result;
    }

  private:
    Context *ctx_;
    uint32_t dtype_;
    int64_t rows_, row_len_;
    Tensor table_;
};

// --------------------------------------------------------------------
// RMSNorm and the fused residual add (cpu.rs:2650-2711, 3652)
// --------------------------------------------------------------------

// x' = x + residual_scale * [rms(branch, w_post, post_eps)], h = rms(x', w, eps).
// Returns {x', h}; `weight` / `w_post` are device f32 [hidden] or nullptr.
inline std::pair<Tensor, Tensor> add_rms(Context &ctx, const Tensor &x, const Tensor *branch,
                                         const Tensor *weight, float eps, const Tensor *w_post = nullptr,
                                         float post_eps = -1.0f, float residual_scale = 1.0f) {
    const int64_t hidden = x.dim(-1), rows = x.numel() / hidden;
    Tensor xo(ctx, x.shape(), x.dtype()), h(ctx, x.shape(), x.dtype());
    ctx.check(cuca_hip_add_rmsnorm(ctx.raw(), x.data(), branch ? branch->data() : nullptr,
                                   weight ? static_cast<const float *>(weight->data()) : nullptr,
                                   w_post ? static_cast<const float *>(w_post->data()) : nullptr, eps,
                                   post_eps < 0 ? eps : post_eps, residual_scale, rows, hidden, xo.data(),
                                   h.data(), (cuca_dtype)x.dtype()));
    return {std::move(xo), std::move(h)};
}

// RMSNorm with a learned weight, no `1 + w` (cpu.rs:3652); nullptr weight is
// the weightless norm (gpu.rs:5895).
inline Tensor rms(Context &ctx, const Tensor &x, const Tensor *weight, float eps) {
    const int64_t hidden = x.dim(-1), rows = x.numel() / hidden;
    Tensor h(ctx, x.shape(), x.dtype());
    ctx.check(cuca_hip_add_rmsnorm(ctx.raw(), x.data(), nullptr,
                                   weight ? static_cast<const float *>(weight->data()) : nullptr, nullptr,
                                   eps, eps, 1.0f, rows, hidden, nullptr, h.data(), (cuca_dtype)x.dtype()));
    return h;
}

// --------------------------------------------------------------------
// Glu (cpu.rs:342-371)
// --------------------------------------------------------------------

struct Glu {
    Act act;
    std::optional<float> clamp;

    explicit Glu(Act a) : act(a) {}
    // `act` with a clamp at `limit` (none when `limit` is not positive).
    static Glu clamped(Act a, float limit) {
        Glu g(a);
        if (limit > 0.0f) g.clamp = limit;
        return g;
    }

    // act(gate) * up over [rows, ff] tensors.
    Tensor apply(Context &ctx, const Tensor &gate, const Tensor &up) const {
        const int64_t ff = gate.dim(-1), rows = gate.numel() / ff;
        Tensor out(ctx, gate.shape(), gate.dtype());
        ctx.check(cuca_hip_glu(ctx.raw(), gate.data(), ff, up.data(), ff, rows, ff, (cuca_act)act,
                               clamp.value_or(0.0f), out.data(), ff, (cuca_dtype)gate.dtype()));
        return out;
    }

    // GateUp::Fused: y [rows, 2 ff] = [gate | up] (cpu.rs:3559-3562).
    Tensor apply_fused(Context &ctx, const Tensor &y, int64_t ff) const {
        const int64_t rows = y.numel() / (2 * ff);
        Tensor out(ctx, {rows, ff}, y.dtype());
        const char *base = static_cast<const char *>(y.data());
        ctx.check(cuca_hip_glu(ctx.raw(), base, 2 * ff, base + ff * dtype_size(y.dtype()), 2 * ff, rows, ff,
                               (cuca_act)act, clamp.value_or(0.0f), out.data(), ff, (cuca_dtype)y.dtype()));
        return out;
    }
};

// --------------------------------------------------------------------
// RoPE (rope.rs, cpu.rs:3672-3688)
// --------------------------------------------------------------------

struct CosSin {
    int32_t half;
    std::vector<float> cos, sin;
};

struct RopeSpec {
    RopeKind kind;
    int32_t n_dims;
    double base;
    double freq_scale = 1.0;
    double yarn_ext_factor = 0.0, yarn_beta_fast = 32.0, yarn_beta_slow = 1.0;
    int64_t yarn_n_ctx_orig = 0;
    double attn_factor = 1.0;

    static RopeSpec plain(RopeKind kind, int32_t n_dims, double base) { return RopeSpec{kind, n_dims, base}; }

    // Row-major [positions, n_dims / 2] tables (rope.rs:136-151).
    CosSin tables(const std::vector<float> *factors, int64_t positions) const {
        cuca_rope_spec s{(int32_t)kind, n_dims, base, freq_scale, yarn_ext_factor, yarn_beta_fast,
                         yarn_beta_slow, yarn_n_ctx_orig, attn_factor};
        CosSin t{n_dims / 2, std::vector<float>((size_t)positions * (n_dims / 2)),
                 std::vector<float>((size_t)positions * (n_dims / 2))};
        if (factors && (int32_t)factors->size() != n_dims / 2)
            throw Error(CUCA_INVALID_ARG, "factors must hold n_dims / 2 values");
        check(nullptr, cuca_hip_rope_tables(&s, factors ? factors->data() : nullptr, positions, t.cos.data(),
                                            t.sin.data()));
        return t;
    }
};

// Rotate the first n_dims values of every head of x [rows, heads, d] in place
// (apply_rope, cpu.rs:3672-3688).  cos/sin: device f32 [table_rows, n_dims/2];
// positions: device int32 [rows]; norm_w: optional fused QK-norm weight [d].
inline void apply_rope(Context &ctx, Tensor &x, const Tensor &cos, const Tensor &sin, RopeKind kind,
                       int32_t n_dims, const Tensor &positions, const Tensor *norm_w = nullptr,
                       float eps = 1e-6f) {
    const int64_t rows = x.dim(0), heads = x.dim(1), d = x.dim(2);
    ctx.check(cuca_hip_rope(ctx.raw(), x.data(), heads * d, nullptr, 0, rows, (int32_t)heads, 0, (int32_t)d,
                            n_dims, (cuca_rope_kind)kind, static_cast<const float *>(cos.data()),
                            static_cast<const float *>(sin.data()), cos.dim(0),
                            static_cast<const int32_t *>(positions.data()),
                            norm_w ? static_cast<const float *>(norm_w->data()) : nullptr, nullptr, eps,
                            (cuca_dtype)x.dtype()));
}

// One K/V-owning layer's paged cache (KvPool, gpu.rs:1774-1781; KvLayer,
// cpu.rs:689-714): keys and values [n_blocks, n_kv_head, 16, head_dim] of
// the activation type, zero-filled.  Position p of a sequence is row p % 16
// of block table[p / 16] (paged.rs:9-16).
class KvPool {
  public:
    KvPool(Context &ctx, int64_t n_blocks, int64_t n_kv_head, int64_t head_dim, DType dtype)
        : n_blocks_(n_blocks), k_(ctx, {n_blocks, n_kv_head, CUCA_KV_BLOCK, head_dim}, dtype),
          v_(ctx, {n_blocks, n_kv_head, CUCA_KV_BLOCK, head_dim}, dtype) {
        std::vector<uint8_t> zeros(k_.bytes(), 0);
        k_.upload(zeros);
        v_.upload(zeros);
    }

    // The pool rows of cache indices start..start+t (host).
    std::vector<int32_t> slots(const std::vector<uint32_t> &table, int64_t start, int64_t t) const {
        std::vector<int32_t> out((size_t)t);
        check(nullptr, cuca_hip_kv_slots(table.data(), (int64_t)table.size(), start, t, n_blocks_,
                                         out.data()));
        return out;
    }

    // store_kv (cpu.rs:3028-3097): q [rows, nq, d] normalised and rotated in
    // place; k normalised, rotated and stored; v (weightless-normalised when
    // v_norm) stored; one launch.  slots: device int32 [rows] from slots().
    void store_kv(Context &ctx, Tensor &q, const Tensor &k, const Tensor &v, const Tensor &cos,
                  const Tensor &sin, RopeKind kind, int32_t n_dims, const Tensor &positions,
                  const Tensor &slots, const Tensor *q_norm_w = nullptr,
                  const Tensor *k_norm_w = nullptr, bool v_norm = false, float eps = 1e-6f) {
        const int64_t rows = q.dim(0), nq = q.dim(1), d = q.dim(2), nk = k.dim(1);
        if (k.shape() != std::vector<int64_t>{rows, nk, d} || v.shape() != k.shape() ||
            nk != k_.dim(1) || d != k_.dim(3))
            throw Error(CUCA_INVALID_ARG, "store_kv: row shape mismatch");
        auto w = [](const Tensor *t) { return t ? static_cast<const float *>(t->data()) : nullptr; };
        ctx.check(cuca_hip_rope_store_kv(
            ctx.raw(), q.data(), nq * d, k.data(), nk * d, v.data(), nk * d, rows, (int32_t)nq,
            (int32_t)nk, (int32_t)d, n_dims, (cuca_rope_kind)kind, static_cast<const float *>(cos.data()),
            static_cast<const float *>(sin.data()), cos.dim(0), static_cast<const int32_t *>(positions.data()),
            w(q_norm_w), w(k_norm_w), v_norm ? 1 : 0, eps, k_.data(), v_.data(), n_blocks_,
            static_cast<const int32_t *>(slots.data()), (cuca_dtype)q.dtype()));
    }

    // Paged decode attention of q [rows, n_head, d] (one query row per
    // sequence) over this pool (paged_attention_decode, paged_kernel.rs:
    // 92-282): tables device u32 [rows, max_blocks], ranges device int32
    // [rows, 2] (lo, hi).  Returns [rows, n_head, d]; the workspace is
    // allocated here (cuca_hip_paged_decode_workspace bytes) unless given.
    Tensor decode(Context &ctx, const Tensor &q, const Tensor &tables, const Tensor &ranges, int32_t n_head,
                  float scale, Tensor *workspace = nullptr) const {
        const int64_t rows = q.dim(0), d = q.dim(2), max_blocks = tables.dim(1);
        if (q.dim(1) != n_head || d != k_.dim(3)) throw Error(CUCA_INVALID_ARG, "attention: query shape mismatch");
        size_t need = 0;
        check(nullptr, cuca_hip_paged_decode_workspace(rows, n_head, (int32_t)d, max_blocks, &need));
        Tensor own;
        if (!workspace) {
            own = Tensor(ctx, {(int64_t)(need > 16 ? need : 16)}, DType::U8);
            workspace = &own;
        }
        Tensor out(ctx, {rows, (int64_t)n_head, d}, q.dtype());
        ctx.check(cuca_hip_paged_decode(ctx.raw(), q.data(), (int64_t)n_head * d, k_.data(), v_.data(), n_blocks_,
                                        static_cast<const uint32_t *>(tables.data()), max_blocks,
                                        static_cast<const int32_t *>(ranges.data()), rows, n_head,
                                        (int32_t)k_.dim(1), (int32_t)d, scale, workspace->data(),
                                        workspace->bytes(), out.data(), (cuca_dtype)q.dtype()));
        ctx.sync(); // the workspace may be freed on return
        return out;
    }

    const Tensor &k() const { return k_; }
    const Tensor &v() const { return v_; }

  private:
    int64_t n_blocks_;
    Tensor k_, v_;
};

}  // namespace cuca
