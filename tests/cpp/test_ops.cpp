// GPU test of the C++ host side (include/cuca_ops.hpp) over the C ABI,
// checked against the CPU oracle (oracle/cuca_oracle.h, test infrastructure).
// Built by __graft_entry__.build(); run by tests/test_gpu_cpp.py.  Prints one
// line per case and exits non-zero on the first failure.
#include "cuca_ops.hpp"

#include "../../oracle/cuca_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>

static int g_fail = 0;
#define EXPECT(cond, ...)                                                                  \
    do {                                                                                   \
        if (!(cond)) {                                                                     \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__);                               \
            std::printf(__VA_ARGS__);                                                      \
            std::printf("\n");                                                             \
            std::fflush(stdout);                                                           \
            std::exit(1);                                                                  \
        }                                                                                  \
    } while (0)

static std::vector<float> normal(std::mt19937 &g, size_t n, float std_ = 1.0f) {
    std::normal_distribution<float> d(0.0f, std_);
    std::vector<float> v(n);
    for (auto &x : v) x = d(g);
    return v;
}

static double max_rel(const std::vector<float> &a, const std::vector<float> &b) {
    double m = 0;
    for (size_t i = 0; i < a.size(); i++) {
        const double den = std::fmax(std::fabs((double)b[i]), 1e-30);
        m = std::fmax(m, std::fabs((double)a[i] - b[i]) / den);
    }
    return m;
}

int main() {
    cuca::Context ctx(0);
    std::mt19937 g(7);

    {  // TokenEmbedding::rows, Q4_0 and Q8_0, bit-exact
        for (uint32_t ty : {(uint32_t)CUCA_GGML_Q4_0, (uint32_t)CUCA_GGML_Q8_0}) {
            const int64_t vocab = 300, hidden = 1024;
            const int64_t rb = oracle_row_bytes(ty, hidden);
            std::vector<uint8_t> table(vocab * rb);
            std::uniform_int_distribution<int> byte(0, 255);
            for (auto &b : table) b = (uint8_t)byte(g);
            for (int64_t blk = 0; blk < vocab * hidden / 32; blk++) {  // finite f16 scales
                const uint16_t d = oracle_f32_to_f16(0.001f + 0.049f * (float)(blk % 97) / 97.0f);
                std::memcpy(&table[blk * (ty == CUCA_GGML_Q4_0 ? 18 : 34)], &d, 2);
            }
            std::vector<uint32_t> ids = {0, 299, 17, 17, 150};
            cuca::TokenEmbedding emb(ctx, ty, table, vocab, hidden);
            const auto got = emb.rows(ids, 1.5f).download<float>();
            std::vector<float> want(ids.size() * hidden);
            int64_t bad = -1;
            EXPECT(oracle_embed(table.data(), ty, vocab, hidden, ids.data(), (int64_t)ids.size(), 1.5f,
                                want.data(), OR_F32, 1, &bad) == 0, "oracle embed");
            EXPECT(std::memcmp(got.data(), want.data(), want.size() * 4) == 0, "embed type %u not bit-exact", ty);
            bool threw = false;
            try {
                (void)emb.rows({1, 300}, 1.0f);
            } catch (const cuca::Error &e) {
                threw = e.status == CUCA_OUT_OF_RANGE &&
                        std::string(e.what()) == "token id 300 outside the embedding table of 300 rows";
            }
            EXPECT(threw, "bad id must raise the reference's error");
        }
        std::printf("ok TokenEmbedding::rows\n");
    }
    {  // add_rms / rms, f32
        const int64_t rows = 9, hidden = 3584;
        auto x = normal(g, rows * hidden, 2.0f), b = normal(g, rows * hidden, 2.0f), w = normal(g, hidden, 0.02f);
        for (auto &v : w) v += 1.0f;
        auto dx = ctx.tensor(x, {rows, hidden}, cuca::DType::F32);
        auto db = ctx.tensor(b, {rows, hidden}, cuca::DType::F32);
        auto dw = ctx.tensor(w, {hidden}, cuca::DType::F32);
        auto [xo, h] = cuca::add_rms(ctx, dx, &db, &dw, 1e-6f);
        std::vector<float> wx(rows * hidden), wh(rows * hidden);
        oracle_add_rmsnorm(x.data(), b.data(), w.data(), nullptr, 1e-6f, 1e-6f, 1.0f, rows, hidden, wx.data(),
                           wh.data(), OR_F32, 1);
        EXPECT(std::memcmp(xo.download<float>().data(), wx.data(), wx.size() * 4) == 0, "x' not bit-exact");
        EXPECT(max_rel(h.download<float>(), wh) <= 1e-5, "h rel err %g", max_rel(h.download<float>(), wh));
        auto h2 = cuca::rms(ctx, dx, &dw, 1e-6f);
        oracle_add_rmsnorm(x.data(), nullptr, w.data(), nullptr, 1e-6f, 1e-6f, 1.0f, rows, hidden, nullptr,
                           wh.data(), OR_F32, 1);
        EXPECT(max_rel(h2.download<float>(), wh) <= 1e-5, "rms rel err");
        std::printf("ok add_rms / rms\n");
    }
    {  // Glu::apply, Glu::clamped, apply_fused
        const int64_t rows = 5, ff = 768;
        auto y = normal(g, rows * 2 * ff);
        auto dy = ctx.tensor(y, {rows, 2 * ff}, cuca::DType::F32);
        auto got = cuca::Glu::clamped(cuca::Act::Silu, 1.5f).apply_fused(ctx, dy, ff).download<float>();
        std::vector<float> want(rows * ff);
        oracle_glu(y.data(), 2 * ff, y.data() + ff, 2 * ff, rows, ff, OR_SILU, 1.5f, want.data(), ff, OR_F32, 1);
        EXPECT(max_rel(got, want) <= 1e-5, "glu rel err %g", max_rel(got, want));
        std::printf("ok Glu\n");
    }
    {  // RopeSpec::tables + apply_rope, NEOX, bit-exact
        const int64_t rows = 6, heads = 4, d = 128;
        auto spec = cuca::RopeSpec::plain(cuca::RopeKind::Neox, (int32_t)d, 1e6);
        auto t = spec.tables(nullptr, 32);
        std::vector<float> oc(t.cos.size()), os(t.sin.size());
        oracle_rope_tables((int)d, 1e6, 1.0, 0.0, 32.0, 1.0, 0, 1.0, nullptr, 32, oc.data(), os.data());
        EXPECT(std::memcmp(t.cos.data(), oc.data(), oc.size() * 4) == 0, "cos table");
        auto x = normal(g, rows * heads * d);
        std::vector<int32_t> pos = {0, 3, 31, 7, 7, 1};
        auto dx = ctx.tensor(x, {rows, heads, d}, cuca::DType::F32);
        auto dc = ctx.tensor(t.cos, {32, d / 2}, cuca::DType::F32);
        auto ds = ctx.tensor(t.sin, {32, d / 2}, cuca::DType::F32);
        auto dp = ctx.tensor(pos, {rows}, cuca::DType::I32);
        cuca::apply_rope(ctx, dx, dc, ds, cuca::RopeKind::Neox, (int32_t)d, dp);
        std::vector<float> want = x;
        oracle_rope(want.data(), heads * d, rows, (int)heads, (int)d, (int)d, OR_ROPE_NEOX, oc.data(), os.data(),
                    pos.data(), nullptr, 1e-6f, OR_F32, 1);
        EXPECT(std::memcmp(dx.download<float>().data(), want.data(), want.size() * 4) == 0, "rope not bit-exact");
        ctx.check_device();
        std::printf("ok RopeSpec::tables / apply_rope\n");
    }
    {  // KvPool::slots + store_kv (NEOX, f32), bit-exact against rope + store_rows
        const int64_t rows = 21, nq = 4, nk = 2, d = 64, n_blocks = 6, start = 9;
        const std::vector<uint32_t> table = {5, 1, 3};
        cuca::KvPool pool(ctx, n_blocks, nk, d, cuca::DType::F32);
        const auto slots = pool.slots(table, start, rows);
        auto spec = cuca::RopeSpec::plain(cuca::RopeKind::Neox, (int32_t)d, 1e4);
        auto t = spec.tables(nullptr, 64);
        auto q = normal(g, rows * nq * d), k = normal(g, rows * nk * d), v = normal(g, rows * nk * d);
        std::vector<int32_t> pos(rows);
        for (int64_t i = 0; i < rows; i++) pos[i] = (int32_t)(start + i);
        auto dq = ctx.tensor(q, {rows, nq, d}, cuca::DType::F32);
        auto dk = ctx.tensor(k, {rows, nk, d}, cuca::DType::F32);
        auto dv = ctx.tensor(v, {rows, nk, d}, cuca::DType::F32);
        auto dc = ctx.tensor(t.cos, {64, d / 2}, cuca::DType::F32);
        auto ds = ctx.tensor(t.sin, {64, d / 2}, cuca::DType::F32);
        auto dp = ctx.tensor(pos, {rows}, cuca::DType::I32);
        auto dsl = ctx.tensor(slots, {rows}, cuca::DType::I32);
        pool.store_kv(ctx, dq, dk, dv, dc, ds, cuca::RopeKind::Neox, (int32_t)d, dp, dsl);
        ctx.check_device();
        std::vector<float> wq = q, wk = k;
        oracle_rope(wq.data(), nq * d, rows, (int)nq, (int)d, (int)d, OR_ROPE_NEOX, t.cos.data(), t.sin.data(),
                    pos.data(), nullptr, 1e-6f, OR_F32, 1);
        oracle_rope(wk.data(), nk * d, rows, (int)nk, (int)d, (int)d, OR_ROPE_NEOX, t.cos.data(), t.sin.data(),
                    pos.data(), nullptr, 1e-6f, OR_F32, 1);
        // store_rows takes [n_kv][rows][d]
        std::vector<float> sk(wk.size()), sv(v.size());
        for (int64_t r = 0; r < rows; r++)
            for (int64_t h = 0; h < nk; h++)
                for (int64_t e = 0; e < d; e++) {
                    sk[(h * rows + r) * d + e] = wk[(r * nk + h) * d + e];
                    sv[(h * rows + r) * d + e] = v[(r * nk + h) * d + e];
                }
        std::vector<float> pk((size_t)(n_blocks * nk * 16 * d), 0.0f), pv = pk;
        EXPECT(oracle_store_rows(table.data(), (int64_t)table.size(), start, rows, sk.data(), pk.data(), n_blocks,
                                 (int)nk, (int)d, OR_F32) == 0, "oracle store k");
        EXPECT(oracle_store_rows(table.data(), (int64_t)table.size(), start, rows, sv.data(), pv.data(), n_blocks,
                                 (int)nk, (int)d, OR_F32) == 0, "oracle store v");
        EXPECT(std::memcmp(dq.download<float>().data(), wq.data(), wq.size() * 4) == 0, "q not bit-exact");
        EXPECT(std::memcmp(pool.k().download<float>().data(), pk.data(), pk.size() * 4) == 0, "pool k");
        EXPECT(std::memcmp(pool.v().download<float>().data(), pv.data(), pv.size() * 4) == 0, "pool v");
        bool threw = false;
        try {
            (void)pool.slots({5, CUCA_NO_BLOCK}, 0, 20);
        } catch (const cuca::Error &e) {
            threw = e.status == CUCA_OUT_OF_RANGE &&
                    std::string(e.what()).find("position 16 has no K/V block") != std::string::npos;
        }
        EXPECT(threw, "a released block must be rejected");
        std::printf("ok KvPool::slots / store_kv\n");

        // decode attention over the stored rows: one query row per position range
        const int64_t qn = 2;
        auto qd = normal(g, qn * nq * d);
        auto dqd = ctx.tensor(qd, {qn, nq, d}, cuca::DType::F32);
        std::vector<uint32_t> tabs = {5, 1, 3, 5, 1, 3};
        std::vector<int32_t> rng = {9, 30, 16, 17};
        auto dt = ctx.tensor(tabs, {qn, 3}, cuca::DType::U32);
        auto dr = ctx.tensor(rng, {qn, 2}, cuca::DType::I32);
        auto got = pool.decode(ctx, dqd, dt, dr, (int32_t)nq, 0.125f).download<float>();
        std::vector<float> want(got.size());
        EXPECT(oracle_paged_attention(qd.data(), qn, (int)nq, (int)nk, (int)d, tabs.data(), 3, rng.data(), pk.data(),
                                      pv.data(), n_blocks, 0.125f, want.data(), OR_F32, 1) == 0,
               "oracle attention");
        double err = 0;  // outputs are convex combinations of N(0, 1) values
        for (size_t i = 0; i < got.size(); i++) err = std::fmax(err, std::fabs((double)got[i] - want[i]));
        EXPECT(err <= 2e-5, "attention abs err %g", err);
        ctx.check_device();
        std::printf("ok KvPool::decode\n");
    }
    {  // errors carry the library's message
        bool threw = false;
        try {
            cuca::Tensor x(ctx, {2, 64}, cuca::DType::F32);
            (void)cuca::Glu(cuca::Act::Silu).apply(ctx, x, x);
            cuca::Tensor bad(ctx, {2, 63}, cuca::DType::F32);
            cuca::RopeSpec::plain(cuca::RopeKind::Norm, 7, 1e4).tables(nullptr, 4);
        } catch (const cuca::Error &e) {
            threw = e.status == CUCA_INVALID_ARG && std::string(e.what()).find("even") != std::string::npos;
        }
        EXPECT(threw, "odd n_dims must be rejected");
        std::printf("ok errors\n");
    }
    std::printf("all ok\n");
    return g_fail;
}
