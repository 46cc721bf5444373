// Checks on the GPU that v_mfma_f32_4x4x1f32 with a -0.0 accumulator returns exactly v_mul_f32's
// rounded product (the fused update kernel's bit-exact engine relies on it): 64 lanes x 4096
// input sets, the 16 blocks' 4x4 outer products compared bit for bit with the vector multiply,
// over ordinary values, zeros of both signs, denormal inputs and denormal products.
// Prints "mismatches M of P products"; exit status 0 when M == 0.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kSets = 4096;

__global__ __launch_bounds__(64) void k_check(const float* a, const float* b, uint32_t* bad) {
    const int l = threadIdx.x;
    uint32_t nb = 0;
    for (int it = 0; it < kSets; ++it) {
        const v4f nz = {-0.0f, -0.0f, -0.0f, -0.0f};
        const v4f d = __builtin_amdgcn_mfma_f32_4x4x1f32(a[it * 64 + l], b[it * 64 + l], nz, 0, 0, 0);
        const int blk = l / 4, n = l % 4;  // lane l holds D[blk][r][n], r = 0..3
        for (int r = 0; r < 4; ++r) {
            const float want = a[it * 64 + blk * 4 + r] * b[it * 64 + blk * 4 + n];
            if (__float_as_uint(want) != __float_as_uint(d[r])) ++nb;
        }
    }
    bad[l] = nb;
}

static uint32_t next(uint64_t* s) {
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(*s >> 32);
}

int main() {
    const int n = kSets * 64;
    float* ha = (float*)malloc(n * sizeof(float));
    float* hb = (float*)malloc(n * sizeof(float));
    uint64_t s = 12345;
    for (int i = 0; i < n; ++i) {
        const float u = (float)(next(&s) % 2001) / 1000.0f - 1.0f, v = (float)(next(&s) % 2001) / 1000.0f - 1.0f;
        float x = ldexpf(u, (int)(next(&s) % 9) - 4), y = ldexpf(v, -(int)(next(&s) % 6));
        switch (i % 8) {
            case 0: x = ldexpf(1.2345f, -130 + i % 20); break;                 // denormal and tiny inputs
            case 1: x = ldexpf(1.3f, -60 - i % 10); y = ldexpf(1.75f, -70); break;  // denormal products
            case 2: x = (i & 16) ? 0.0f : -0.0f; break;                        // zeros of both signs
            case 3: y = (i & 32) ? 0.0f : -0.0f; break;
            default: break;
        }
        ha[i] = x;
        hb[i] = y;
    }
    float *da = nullptr, *db = nullptr;
    uint32_t* dbad = nullptr;
    if (hipMalloc(&da, n * sizeof(float)) != hipSuccess || hipMalloc(&db, n * sizeof(float)) != hipSuccess ||
        hipMalloc(&dbad, 64 * sizeof(uint32_t)) != hipSuccess) {
        fprintf(stderr, "allocation failed\n");
        return 2;
    }
    if (hipMemcpy(da, ha, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(db, hb, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
        fprintf(stderr, "copy failed\n");
        return 2;
    }
    hipLaunchKernelGGL(k_check, dim3(1), dim3(64), 0, 0, da, db, dbad);
    uint32_t bad[64];
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(bad, dbad, sizeof bad, hipMemcpyDeviceToHost) != hipSuccess) {
        fprintf(stderr, "kernel failed\n");
        return 2;
    }
    uint64_t total = 0;
    for (int l = 0; l < 64; ++l) total += bad[l];
    printf("mismatches %llu of %d products\n", (unsigned long long)total, kSets * 256);
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(dbad);
    free(ha);
    free(hb);
    return total == 0 ? 0 : 1;
}
