// Streaming-read rate on the running GPU: the practical ceiling the single-token
// decode step (which reads every weight byte of two experts once) is measured
// against.  Each launch reads a contiguous buffer once with 16-byte loads, one
// 1024-thread block per CU (or two), every lane keeping U loads in flight; the
// table gives microseconds per launch (back-to-back launches, hipEvent over
// the run) and the rate.  "resident" reads the same buffer every launch (it
// stays in the 256 MB last-level cache when it fits); "cycled" rotates over six
// buffers (1.2 GB in all), so each launch reads bytes last touched six launches
// earlier, i.e. from HBM.
//
//   jxai_amd/probe/hbm_stream          (built by python -m jxai_amd.build)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                                   \
    do {                                                                           \
        hipError_t e_ = (x);                                                       \
        if (e_ != hipSuccess) {                                                    \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            exit(1);                                                               \
        }                                                                          \
    } while (0)

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Block b reads vectors [b * per_block, (b + 1) * per_block) of buf, per_block a
// multiple of 1024 * U; the xor of what each lane read goes to out (so no load is dead).
template <int U, bool NT>
__global__ void __launch_bounds__(1024) k_stream(const u32x4* __restrict__ buf, size_t per_block, unsigned* out) {
    const u32x4* p = buf + (size_t)blockIdx.x * per_block + threadIdx.x;
    unsigned acc = 0;
    for (size_t it = 0; it < per_block; it += 1024 * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(p + it + u * 1024) : p[it + u * 1024];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    out[(size_t)blockIdx.x * 1024 + threadIdx.x] = acc;
}

constexpr int NBUF = 6;
constexpr int REPS = 200;

template <int U, bool NT>
static void run(const u32x4* base, size_t buf_vecs, size_t bytes, int blocks, bool cycled, unsigned* out) {
    const size_t per_block = bytes / 16 / blocks / (1024 * U) * (1024 * U);
    auto launch = [&](int i) {
        const u32x4* b = base + (cycled ? (size_t)(i % NBUF) * buf_vecs : 0);
        hipLaunchKernelGGL((k_stream<U, NT>), dim3(blocks), dim3(1024), 0, 0, b, per_block, out);
    };
    for (int i = 0; i < 2 * NBUF; ++i) launch(i);
    hipEvent_t t0, t1;
    CHECK(hipEventCreate(&t0));
    CHECK(hipEventCreate(&t1));
    CHECK(hipEventRecord(t0));
    for (int i = 0; i < REPS; ++i) launch(i);
    CHECK(hipEventRecord(t1));
    CHECK(hipEventSynchronize(t1));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, t0, t1));
    CHECK(hipEventDestroy(t0));
    CHECK(hipEventDestroy(t1));
    const double moved = (double)per_block * blocks * 16, us = ms * 1e3 / REPS;
    printf("%6.1f MB  %-8s  %4d blocks  %d x 16 B in flight per lane%-16s  %7.2f us/launch  %5.2f TB/s\n",
           moved / 1e6, cycled ? "cycled" : "resident", blocks, U, NT ? " (non-temporal)" : "", us,
           moved / us / 1e6);
    fflush(stdout);
}

int main() {
    int ncu = 0;
    CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
    const size_t MB = 1 << 20, max_bytes = 198 * MB, buf_vecs = max_bytes / 16;
    u32x4* buf = nullptr;
    unsigned* out = nullptr;
    CHECK(hipMalloc(&buf, max_bytes * NBUF));
    CHECK(hipMemset(buf, 0x5a, max_bytes * NBUF));
    CHECK(hipMalloc(&out, (size_t)2 * ncu * 1024 * sizeof(unsigned)));
    printf("streaming reads, %d CUs, %d back-to-back launches per row\n", ncu, REPS);
    for (size_t bytes : {132 * MB, 198 * MB}) {  // one layer's gate/up bytes; its gate/up/down bytes
        for (bool cycled : {false, true}) {
            run<1, false>(buf, buf_vecs, bytes, ncu, cycled, out);
            run<2, false>(buf, buf_vecs, bytes, ncu, cycled, out);
            run<4, false>(buf, buf_vecs, bytes, ncu, cycled, out);
            run<8, false>(buf, buf_vecs, bytes, ncu, cycled, out);
            run<4, true>(buf, buf_vecs, bytes, ncu, cycled, out);
            run<4, false>(buf, buf_vecs, bytes, 2 * ncu, cycled, out);
        }
    }
    CHECK(hipDeviceSynchronize());
    CHECK(hipFree(buf));
    CHECK(hipFree(out));
    return 0;
}
