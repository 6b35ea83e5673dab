// probe-links: biv_hip oracle
//
// The C++ host mirror (include/biv_hip.hpp) on the GPU, against the CPU
// oracle (oracle/oracle.c, linked as the checker only), written as biv's own
// tests of the block would be: a 32-expert Q8_0 layer with a shared expert
// (n_embd 1024, n_ff 512, k 8) from seeded N(0, 0.02) weights.
//   - DeviceMoe::ffn (Model::ffn) bit-identical to the oracle's Model::moe at
//     T = 1 and 5 (decode kernels), within 1e-3 * RMS at T = 64 (matrix-core
//     down), and the same bits on a second call;
//   - ffn_add is x + ffn(h) (the residual add, model.rs:788-790), encode on
//     device buffers gives the ffn's bits;
//   - DeviceDense::ffn (dense_ffn, model.rs:1118-1126) bit-identical;
//   - failures as Error with the library's code: an unsupported type
//     (Error::NoKernel -> BIV_HIP_E_TYPE), mismatched shapes
//     (Error::TensorShape -> BIV_HIP_E_INVALID).
// Prints one line per check and "host mirror: N failures"; exits 1 on any.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/biv_hip.hpp"

using namespace biv::hip;

// the oracle's C entry points (oracle/oracle.c)
extern "C" {
typedef struct {
    int32_t ty, pad;
    const uint8_t *data;
    uint64_t stride, offset;
} OrcExperts;
typedef struct {
    int32_t ty, pad;
    const uint8_t *data;
} OrcWeight;
typedef struct {
    int32_t n_expert, k, n_embd, n_ff, n_ff_sh, pad;
    OrcWeight router;
    OrcExperts gate, up, down;
    OrcWeight sh_gate, sh_up, sh_down, gate_inp;
} OrcMoe;
int orc_moe(const OrcMoe *m, const float *h, size_t n, float *out, int threads, int level, int32_t *ids_out,
            float *w_out, float *logits_out);
int orc_dense_ffn(int gty, const uint8_t *gate, int uty, const uint8_t *up, int dty, const uint8_t *down, size_t e,
                  size_t ff, const float *x, size_t n, float *out, int threads, int level);
}

static int failures = 0;
static void check(bool ok, const char *what)
{
    printf("%s: %s\n", what, ok ? "ok" : "FAILED");
    if (!ok) failures++;
}

// SplitMix64 and Box-Muller: seeded N(0, 1)
struct Rng {
    uint64_t s;
    uint64_t next()
    {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uni() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    float normal() { return (float)(std::sqrt(-2.0 * std::log(uni())) * std::cos(6.283185307179586 * uni())); }
};

// rows x cols of N(0, std) quantised to Q8_0 (d = amax / 127 as f16, q = round(x / d))
static std::vector<uint8_t> q8_matrix(Rng &r, size_t rows, size_t cols, float std)
{
    std::vector<uint8_t> out(rows * row_size(GgmlType::Q8_0, cols));
    uint8_t *p = out.data();
    for (size_t i = 0; i < rows; i++)
        for (size_t b = 0; b < cols / 32; b++, p += 34) {
            float v[32], amax = 0.0f;
            for (int j = 0; j < 32; j++) {
                v[j] = std * r.normal();
                amax = std::fmax(amax, std::fabs(v[j]));
            }
            const _Float16 d16 = (_Float16)(amax / 127.0f);
            const float d = (float)d16, id = d != 0.0f ? 1.0f / d : 0.0f;
            std::memcpy(p, &d16, 2);
            for (int j = 0; j < 32; j++) {
                const float q = std::round(v[j] * id);
                p[2 + j] = (uint8_t)(int8_t)std::fmax(-127.0f, std::fmin(127.0f, q));
            }
        }
    return out;
}

static std::vector<uint8_t> f32_matrix(Rng &r, size_t rows, size_t cols, float std)
{
    std::vector<float> v(rows * cols);
    for (auto &x : v) x = std * r.normal();
    std::vector<uint8_t> out(v.size() * 4);
    std::memcpy(out.data(), v.data(), out.size());
    return out;
}

static bool same_bits(const std::vector<float> &a, const std::vector<float> &b)
{
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
}

static double rel_err(const std::vector<float> &ref, const std::vector<float> &got)
{
    double ss = 0.0, mx = 0.0;
    for (size_t i = 0; i < ref.size(); i++) {
        ss += (double)ref[i] * ref[i];
        mx = std::fmax(mx, std::fabs((double)ref[i] - got[i]));
    }
    return mx / std::sqrt(ss / ref.size());
}

int main()
{
    const size_t E = 1024, NE = 32, FF = 512;
    const int K = 8;
    Rng r{42};
    auto router = f32_matrix(r, NE, E, 0.02f);
    auto gate = q8_matrix(r, NE * FF, E, 0.02f), up = q8_matrix(r, NE * FF, E, 0.02f);
    auto down = q8_matrix(r, NE * E, FF, 0.02f);
    auto sg = q8_matrix(r, FF, E, 0.02f), su = q8_matrix(r, FF, E, 0.02f), sd = q8_matrix(r, E, FF, 0.02f);
    auto gi = f32_matrix(r, 1, E, 0.02f);
    const size_t gstride = FF * row_size(GgmlType::Q8_0, E), dstride = E * row_size(GgmlType::Q8_0, FF);

    SharedExpert shared{{GgmlType::Q8_0, E, FF, sg.data()},
                        {GgmlType::Q8_0, E, FF, su.data()},
                        {GgmlType::Q8_0, FF, E, sd.data()},
                        {GgmlType::F32, E, 1, gi.data()}};
    Moe m{{GgmlType::F32, E, NE, router.data()},
          {GgmlType::Q8_0, E, FF, NE, gate.data(), gstride, 0},
          {GgmlType::Q8_0, E, FF, NE, up.data(), gstride, 0},
          {GgmlType::Q8_0, FF, E, NE, down.data(), dstride, 0},
          &shared,
          K};
    OrcMoe om{};
    om.n_expert = (int32_t)NE;
    om.k = K;
    om.n_embd = (int32_t)E;
    om.n_ff = (int32_t)FF;
    om.n_ff_sh = (int32_t)FF;
    om.router = {BIV_GGML_F32, 0, router.data()};
    om.gate = {BIV_GGML_Q8_0, 0, gate.data(), gstride, 0};
    om.up = {BIV_GGML_Q8_0, 0, up.data(), gstride, 0};
    om.down = {BIV_GGML_Q8_0, 0, down.data(), dstride, 0};
    om.sh_gate = {BIV_GGML_Q8_0, 0, sg.data()};
    om.sh_up = {BIV_GGML_Q8_0, 0, su.data()};
    om.sh_down = {BIV_GGML_Q8_0, 0, sd.data()};
    om.gate_inp = {BIV_GGML_F32, 0, gi.data()};

    try {
        Engine eng(0);
        DeviceMoe dm = eng.moe(m);
        printf("%s\n", eng.description().c_str());
        check(!eng.numerics().empty(), "numerics pairs");
        for (size_t T : {1, 5, 64}) {
            std::vector<float> h(T * E);
            for (auto &x : h) x = r.normal();
            std::vector<float> ref(T * E);
            check(orc_moe(&om, h.data(), T, ref.data(), 8, -1, nullptr, nullptr, nullptr) == 0, "oracle moe");
            const std::vector<float> got = dm.ffn(h.data(), T), again = dm.ffn(h.data(), T);
            char what[96];
            if (T < 64) {
                snprintf(what, sizeof what, "T=%zu ffn bit-identical to the oracle", T);
                check(same_bits(ref, got), what);
            }
            const double rel = rel_err(ref, got);
            snprintf(what, sizeof what, "T=%zu ffn max|d|/RMS %.2e <= 1e-3", T, rel);
            check(rel <= 1e-3, what);
            snprintf(what, sizeof what, "T=%zu same bits run to run", T);
            check(same_bits(got, again), what);
            // the residual form and the device form
            std::vector<float> x(T * E), want(T * E);
            for (size_t i = 0; i < x.size(); i++) {
                x[i] = r.normal();
                want[i] = x[i] + got[i];
            }
            dm.ffn_add(h.data(), T, x.data());
            snprintf(what, sizeof what, "T=%zu ffn_add is x + ffn(h)", T);
            check(same_bits(x, want), what);
            float *hd = static_cast<float *>(eng.malloc(h.size() * 4)), *od = static_cast<float *>(eng.malloc(h.size() * 4));
            eng.h2d(hd, h.data(), h.size() * 4);
            dm.encode(hd, T, od, false);
            std::vector<float> dev(T * E);
            eng.d2h(dev.data(), od, dev.size() * 4);
            eng.free(hd);
            eng.free(od);
            snprintf(what, sizeof what, "T=%zu encode (device buffers) gives the ffn's bits", T);
            check(same_bits(dev, got), what);
        }
        // Ffn::Dense
        {
            const size_t DF = 1536;
            auto dg = q8_matrix(r, DF, E, 0.02f), du = q8_matrix(r, DF, E, 0.02f), dd = q8_matrix(r, E, DF, 0.02f);
            DeviceDense dn = eng.dense({GgmlType::Q8_0, E, DF, dg.data()}, {GgmlType::Q8_0, E, DF, du.data()},
                                       {GgmlType::Q8_0, DF, E, dd.data()});
            std::vector<float> h(3 * E), ref(3 * E);
            for (auto &x : h) x = r.normal();
            orc_dense_ffn(BIV_GGML_Q8_0, dg.data(), BIV_GGML_Q8_0, du.data(), BIV_GGML_Q8_0, dd.data(), E, DF,
                          h.data(), 3, ref.data(), 8, -1);
            check(same_bits(dn.ffn(h.data(), 3), ref), "dense ffn bit-identical to the oracle");
        }
        // errors as Error::NoKernel / Error::TensorShape
        {
            int code = 0;
            try {
                eng.weight({static_cast<GgmlType>(99), E, FF, sg.data()});
            } catch (const Error &e) {
                code = e.code();
                printf("  (%s)\n", e.what());
            }
            check(code == BIV_HIP_E_TYPE, "unsupported type throws Error(BIV_HIP_E_TYPE)");
            Moe bad = m;
            bad.down.rows = E / 2; // down no longer n_embd rows
            code = 0;
            try {
                eng.moe(bad);
            } catch (const Error &e) {
                code = e.code();
                printf("  (%s)\n", e.what());
            }
            check(code == BIV_HIP_E_INVALID, "mismatched shapes throw Error(BIV_HIP_E_INVALID)");
        }
    } catch (const Error &e) {
        printf("unexpected Error %d: %s\n", e.code(), e.what());
        failures++;
    }
    printf("host mirror: %d failures\n", failures);
    return failures ? 1 : 0;
}
