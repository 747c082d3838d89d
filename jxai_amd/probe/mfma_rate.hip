// Matrix-core issue rate on the running GPU: the ceiling the prefill GEMMs are
// measured against.  Every kernel keeps NACC independent accumulators per wave
// (so the matrix pipe never waits on a result) and runs ITERS rounds; the
// table gives ns per MFMA per SIMD, the rate as TFLOP/s (TOPS for int8) over
// the whole device, and the shader clock from s_memtime against wall time.
// Variants:
//   operands   random (bit patterns from a hash of the lane) or constant
//   VALU       n independent v_mul_f32 per MFMA, or n v_mul_f32 on the
//              accumulator elements between MFMAs (the prefill GEMM's per-block
//              rescale pattern: 16 multiplies per 32x32 tile)
//   occupancy  1 or 2 waves per SIMD
//
//   jxai_amd/probe/mfma_rate          (built by python -m jxai_amd.build)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int NACC = 8;

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    return x ^ (x >> 16);
}

// MODE 0: independent VALU, MODE 1: VALU on the accumulators (rescale pattern)
template <bool I8, int NV, int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_rate(float* out, int iters, int random, unsigned long long* clk) {
    const uint32_t s = random ? mix(threadIdx.x * 2654435761u + blockIdx.x) : 0x3c003c00u;
    uint32_t w[4];
    for (int i = 0; i < 4; ++i) w[i] = random ? (mix(s + i) & 0x3bff3bffu) : s;  // fp16 below 1.0, no inf/nan
    const h8 a = __builtin_bit_cast(h8, make_uint4(w[0], w[1], w[2], w[3]));
    const h8 b = __builtin_bit_cast(h8, make_uint4(w[3], w[2], w[1], w[0]));
    const v4i ia = __builtin_bit_cast(v4i, make_uint4(w[0], w[1], w[2], w[3]));
    const v4i ib = __builtin_bit_cast(v4i, make_uint4(w[2], w[3], w[0], w[1]));
    constexpr int NF = I8 ? 1 : NACC, NI = I8 ? NACC : 1;  // only the accumulators the variant uses
    v16f acc[NF];
    v16i iacc[NI];
    for (int k = 0; k < NF; ++k) acc[k] = v16f{};
    for (int k = 0; k < NI; ++k) iacc[k] = v16i{};
    float x[8];
    for (int k = 0; k < 8; ++k) x[k] = 1.0f + 1e-3f * (float)(threadIdx.x + k);
    const float r = random ? 0.9999f : 1.0f;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int k = 0; k < NACC; ++k) {
            if constexpr (I8)
                iacc[k % NI] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ia, ib, iacc[k % NI], 0, 0, 0);
            else
                acc[k % NF] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[k % NF], 0, 0, 0);
            if constexpr (MODE == 0) {
#pragma unroll
                for (int v = 0; v < NV; ++v) x[v & 7] *= r;
            } else {  // multiply NV elements of the accumulator issued two MFMAs ago
#pragma unroll
                for (int v = 0; v < NV; ++v) acc[(k + NF - 2) % NF][v & 15] *= r;
            }
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float sum = 0.0f;
    for (int k = 0; k < NF; ++k)
        for (int e = 0; e < 16; ++e) sum += acc[k][e];
    for (int k = 0; k < NI; ++k)
        for (int e = 0; e < 16; ++e) sum += (float)iacc[k][e];
    for (int k = 0; k < 8; ++k) sum += x[k];
    out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
    if (threadIdx.x == 0 && blockIdx.x == 0) *clk = t1 - t0;
}

static int cus() {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || n <= 0) n = 256;
    return n;
}

#define CHECK(x)                                                                 \
    do {                                                                         \
        hipError_t e_ = (x);                                                     \
        if (e_ != hipSuccess) {                                                  \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));         \
            std::exit(1);                                                        \
        }                                                                        \
    } while (0)

template <bool I8, int NV, int MODE>
static void run(const char* name, int waves_per_simd, int random, float* out, unsigned long long* clk) {
    const int iters = 4096;
    const int blocks = cus() * waves_per_simd;  // 4 waves per block: one per SIMD of a CU
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    hipLaunchKernelGGL((k_rate<I8, NV, MODE>), dim3(blocks), dim3(256), 0, 0, out, 64, random, clk);  // warm-up
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL((k_rate<I8, NV, MODE>), dim3(blocks), dim3(256), 0, 0, out, iters, random, clk);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    unsigned long long cycles = 0;
    CHECK(hipMemcpy(&cycles, clk, sizeof(cycles), hipMemcpyDeviceToHost));
    const double mfma_per_simd = (double)waves_per_simd * iters * NACC;
    const double ns = ms * 1e6 / mfma_per_simd;
    const double ops = (double)blocks * 4 * iters * NACC * (I8 ? 65536.0 : 32768.0);
    std::printf("%-34s %-8s %d wave/SIMD  %6.2f ns/MFMA/SIMD  %7.1f %s  clock %.2f GHz\n", name,
                random ? "random" : "const", waves_per_simd, ns, ops / ms / 1e9, I8 ? "TOPS" : "TFLOP/s",
                (double)cycles / (ms * 1e6));
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
}

int main() {
    float* out = nullptr;
    unsigned long long* clk = nullptr;
    CHECK(hipMalloc(&out, (size_t)cus() * 2 * 256 * sizeof(float)));
    CHECK(hipMalloc(&clk, sizeof(unsigned long long)));
    std::printf("v_mfma_f32_32x32x16_f16 (32768 flop) and v_mfma_i32_32x32x32_i8 (65536 op), %d accumulators per wave, "
                "%d CUs\n", NACC, cus());
    for (int rnd = 0; rnd < 2; ++rnd) {
        run<false, 0, 0>("f16 mfma only", 1, rnd, out, clk);
        run<false, 0, 0>("f16 mfma only", 2, rnd, out, clk);
        run<true, 0, 0>("i8 mfma only", 1, rnd, out, clk);
        run<true, 0, 0>("i8 mfma only", 2, rnd, out, clk);
    }
    run<false, 4, 0>("f16 + 4 independent VALU/MFMA", 1, 1, out, clk);
    run<false, 8, 0>("f16 + 8 independent VALU/MFMA", 1, 1, out, clk);
    run<false, 12, 0>("f16 + 12 independent VALU/MFMA", 1, 1, out, clk);
    run<false, 16, 0>("f16 + 16 independent VALU/MFMA", 1, 1, out, clk);
    run<false, 8, 0>("f16 + 8 independent VALU/MFMA", 2, 1, out, clk);
    run<false, 16, 0>("f16 + 16 independent VALU/MFMA", 2, 1, out, clk);
    run<false, 4, 1>("f16 + 4 acc multiplies/MFMA", 1, 1, out, clk);
    run<false, 8, 1>("f16 + 8 acc multiplies/MFMA", 1, 1, out, clk);
    run<false, 8, 1>("f16 + 8 acc multiplies/MFMA", 2, 1, out, clk);
    run<false, 16, 1>("f16 + 16 acc multiplies/MFMA", 2, 1, out, clk);
    CHECK(hipFree(out));
    CHECK(hipFree(clk));
    return 0;
}
