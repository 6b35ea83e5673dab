// Checks, on the GPU, the fact the prefill router rests on: a k = 1 f32
// MFMA block (v_mfma_f32_32x32x1f32, 16x16x1f32, 4x4x1f32: one product per
// output) computes every output as fmaf(a, b, c), a single rounding.  The
// operand and output layouts are read off the instruction first (lane
// indices as values), then random triples are compared bit for bit with
// the host's fmaf: wide exponent ranges, products cancelling c, subnormal
// products, results and accumulators.  Prints one line per instruction and
// exits 1 if any output differs.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// mode 0: 32x32x1 (2 blocks, 32 outputs per lane), 1: 16x16x1 (4 blocks,
// 16), 2: 4x4x1 (16 blocks, 4); C and D hold 32 floats per lane
__global__ void k_mfma(const float *A, const float *B, const float *C, float *D, int mode)
{
    const int l = threadIdx.x;
    const size_t w = blockIdx.x;
    const float a = A[w * 64 + l], b = B[w * 64 + l];
    const float *c = C + (w * 64 + l) * 32;
    float *d = D + (w * 64 + l) * 32;
    if (mode == 0) {
        f32x32 x;
        for (int i = 0; i < 32; i++) x[i] = c[i];
        x = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, x, 0, 0, 0);
        for (int i = 0; i < 32; i++) d[i] = x[i];
    } else if (mode == 1) {
        f32x16 x;
        for (int i = 0; i < 16; i++) x[i] = c[i];
        x = __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, x, 0, 0, 0);
        for (int i = 0; i < 16; i++) d[i] = x[i];
    } else {
        f32x4 x;
        for (int i = 0; i < 4; i++) x[i] = c[i];
        x = __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, x, 0, 0, 0);
        for (int i = 0; i < 4; i++) d[i] = x[i];
    }
}

static float from_bits(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

#define CHECK(x)                                                                                                  \
    do {                                                                                                          \
        hipError_t e_ = (x);                                                                                      \
        if (e_ != hipSuccess) {                                                                                   \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                                             \
            return 2;                                                                                             \
        }                                                                                                         \
    } while (0)

int main()
{
    const int W = 2048, NR[3] = {32, 16, 4};
    const char *name[3] = {"v_mfma_f32_32x32x1f32", "v_mfma_f32_16x16x1f32", "v_mfma_f32_4x4x1f32"};
    const size_t na = (size_t)W * 64, nc = na * 32;
    std::vector<float> hA(na), hB(na), hC(nc), hD(nc);
    float *dA, *dB, *dC, *dD;
    CHECK(hipMalloc(&dA, na * 4));
    CHECK(hipMalloc(&dB, na * 4));
    CHECK(hipMalloc(&dC, nc * 4));
    CHECK(hipMalloc(&dD, nc * 4));
    std::mt19937 rng(1);
    long total_bad = 0;
    for (int mode = 0; mode < 3; mode++) {
        const int nr = NR[mode];
        // layout: wave 0 A = lane + 1, B = 1; wave 1 A = 1, B = lane + 1
        std::fill(hC.begin(), hC.end(), 0.0f);
        for (int l = 0; l < 64; l++) {
            hA[l] = (float)(l + 1), hB[l] = 1.0f;
            hA[64 + l] = 1.0f, hB[64 + l] = (float)(l + 1);
        }
        CHECK(hipMemcpy(dA, hA.data(), 128 * 4, hipMemcpyHostToDevice));
        CHECK(hipMemcpy(dB, hB.data(), 128 * 4, hipMemcpyHostToDevice));
        CHECK(hipMemcpy(dC, hC.data(), 128 * 32 * 4, hipMemcpyHostToDevice));
        k_mfma<<<2, 64>>>(dA, dB, dC, dD, mode);
        CHECK(hipMemcpy(hD.data(), dD, 128 * 32 * 4, hipMemcpyDeviceToHost));
        static int la[64][32], lb[64][32];
        for (int l = 0; l < 64; l++)
            for (int r = 0; r < nr; r++) {
                la[l][r] = (int)hD[l * 32 + r] - 1;
                lb[l][r] = (int)hD[(64 + l) * 32 + r] - 1;
                if (la[l][r] < 0 || la[l][r] > 63 || lb[l][r] < 0 || lb[l][r] > 63) {
                    printf("%s: layout not read (lane %d reg %d)\n", name[mode], l, r);
                    return 1;
                }
            }
        long bad = 0, n = 0;
        for (int trial = 0; trial < 3; trial++) {
            for (size_t i = 0; i < na; i++) {
                int e1, e2;
                if (trial == 0) e1 = 100 + rng() % 56, e2 = 100 + rng() % 56;     // |a b| about 2^-54 .. 2^56
                else if (trial == 1) e1 = 1 + rng() % 60, e2 = 1 + rng() % 60;   // tiny: subnormal products
                else e1 = 117 + rng() % 20, e2 = 117 + rng() % 20;               // around 1
                hA[i] = from_bits((rng() & 0x807fffffu) | ((uint32_t)e1 << 23));
                hB[i] = from_bits((rng() & 0x807fffffu) | ((uint32_t)e2 << 23));
            }
            for (int w = 0; w < W; w++)
                for (int l = 0; l < 64; l++)
                    for (int r = 0; r < nr; r++) {
                        const float p = hA[w * 64 + la[l][r]] * hB[w * 64 + lb[l][r]];
                        const uint32_t u = bits(p);
                        // half of c cancels the product to a few bits, half is of its size
                        float c = (rng() & 1) ? -from_bits(u ^ (rng() & 0xff))
                                              : from_bits((rng() & 0x807fffffu) | (u & 0x7f800000u));
                        if (trial == 1 && (rng() & 3) == 0) c = from_bits(rng() & 0x807fffffu); // subnormal c
                        hC[((size_t)w * 64 + l) * 32 + r] = c;
                    }
            CHECK(hipMemcpy(dA, hA.data(), na * 4, hipMemcpyHostToDevice));
            CHECK(hipMemcpy(dB, hB.data(), na * 4, hipMemcpyHostToDevice));
            CHECK(hipMemcpy(dC, hC.data(), nc * 4, hipMemcpyHostToDevice));
            k_mfma<<<W, 64>>>(dA, dB, dC, dD, mode);
            CHECK(hipGetLastError());
            CHECK(hipMemcpy(hD.data(), dD, nc * 4, hipMemcpyDeviceToHost));
            for (int w = 0; w < W; w++)
                for (int l = 0; l < 64; l++)
                    for (int r = 0; r < nr; r++) {
                        const size_t o = ((size_t)w * 64 + l) * 32 + r;
                        const float want = fmaf(hA[w * 64 + la[l][r]], hB[w * 64 + lb[l][r]], hC[o]);
                        n++;
                        if (bits(want) != bits(hD[o]) && !(want != want && hD[o] != hD[o])) {
                            if (bad < 4)
                                printf("  %s: a=%a b=%a c=%a fmaf=%a mfma=%a\n", name[mode], hA[w * 64 + la[l][r]],
                                       hB[w * 64 + lb[l][r]], hC[o], want, hD[o]);
                            bad++;
                        }
                    }
        }
        printf("%s: %ld of %ld outputs differ from fmaf\n", name[mode], bad, n);
        total_bad += bad;
    }
    return total_bad ? 1 : 0;
}
