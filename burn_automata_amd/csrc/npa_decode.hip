// npa_decode.hip - Gaussian decode and tile-binned 2D splat on gfx950.
//
// decode_gaussians_3d  crates/burn_automata_kernels/src/gaussian.rs:53-223: a per-particle map.
//
// splat_particles_2d   crates/burn_automata_kernels/src/splat.rs:30-93, as a deterministic
// tile-binned rasteriser:
//   k_splat_prep   per particle: pixel-space centre, the in-bounds window weight sum
//                  (the normaliser), colour, and how many 16x16 screen tiles the
//                  (2r+1)^2 window touches;
//   k_scan_1block  exclusive prefix of the per-particle tile counts;
//   k_splat_emit   one (tile, particle) item per touched tile, in particle order;
//   stable key sort of the items by tile (the hashgrid's counting sort) -> per-tile
//                  particle lists in ascending particle index;
//   k_splat_tiles  one 256-thread block per tile, one pixel per thread: the tile's list
//                  is staged through LDS 256 particles at a time and each pixel adds its
//                  weights in list order - the order the reference's serial loop adds them.
#include <hip/hip_runtime.h>

#include "npa_internal.hpp"

namespace npa {

// --------------------------------------------------------------- decode
__global__ __launch_bounds__(256) void k_decode(const float4* __restrict__ pos, const float* __restrict__ states,
                                                uint32_t count, uint32_t S, npa_gaussian_decode_cfg cfg,
                                                uint32_t K, float* __restrict__ pv, float* __restrict__ sh,
                                                float* __restrict__ rot, float* __restrict__ so) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= count) return;
    const float* s = states + (uint64_t)idx * S;
    const float4 p = pos[idx];
    const uint32_t color_start = cfg.mode == NPA_DECODE_SH0_ORIENTED ? S - K * 3 : S - 3;
    for (uint32_t k = 0; k < K; ++k) {  // decode_sh gaussian.rs:134-158
        const uint32_t base = color_start + k * 3;
        for (int ch = 0; ch < 3; ++ch)
            sh[((uint64_t)idx * K + k) * 3 + ch] = clampf_(s[base + ch] + 0.5f, 0.0f, 1.0f);
    }
    float q[4] = {1.0f, 0.0f, 0.0f, 0.0f};
    if (cfg.mode == NPA_DECODE_SH0_ORIENTED) {  // normalize_quat gaussian.rs:214-223
        const uint32_t rs = color_start - 4;
        q[0] = s[rs];
        q[1] = s[rs + 1];
        q[2] = s[rs + 2];
        q[3] = s[rs + 3];
        const float norm = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
        if (norm <= 1e-8f) {
            q[0] = 1.0f;
            q[1] = q[2] = q[3] = 0.0f;
        } else {
            for (int k = 0; k < 4; ++k) q[k] /= norm;
        }
    }
    float o[4];
    switch (cfg.mode) {  // decode_scale_opacity gaussian.rs:160-208
        case NPA_DECODE_PARTICLE_POINT: {
            const float sc = fmaxf(cfg.min_scale, 1.0e-6f);
            o[0] = o[1] = o[2] = sc;
            o[3] = 1.0f;
        } break;
        case NPA_DECODE_SH0_FIXED_SCALE: {
            const float sc = clampf_(cfg.sigma, cfg.min_scale, cfg.max_scale);
            o[0] = o[1] = o[2] = sc;
            o[3] = clampf_(cfg.opacity_scale, cfg.min_opacity, cfg.max_opacity);
        } break;
        case NPA_DECODE_SH0_LEARNED_SCALE: {
            const float scale_logit = clampf_(s[S - 5], -8.0f, 8.0f);
            const float opacity_logit = clampf_(s[S - 4], -12.0f, 12.0f);
            const float sc = clampf_(cfg.sigma * expf(scale_logit), cfg.min_scale, cfg.max_scale);
            const float sig = 1.0f / (1.0f + expf(-opacity_logit));
            const float op = clampf_(sig, cfg.min_opacity, cfg.max_opacity) * cfg.opacity_scale;
            o[0] = o[1] = o[2] = sc;
            o[3] = clampf_(op, cfg.min_opacity, cfg.max_opacity);
        } break;
        default: {
            const uint32_t anis = color_start - 8;
            const float ma = fmaxf(cfg.max_anisotropy, 1e-6f);
            const float ax = tanhf(s[anis] / ma) * cfg.max_anisotropy;
            const float ay = tanhf(s[anis + 1] / ma) * cfg.max_anisotropy;
            const float az = tanhf(s[anis + 2] / ma) * cfg.max_anisotropy;
            const float ol = tanhf(s[anis + 3] / ma) * cfg.max_anisotropy;
            o[0] = clampf_(cfg.sigma * expf(ax), cfg.min_scale, cfg.max_scale);
            o[1] = clampf_(cfg.sigma * expf(ay), cfg.min_scale, cfg.max_scale);
            o[2] = clampf_(cfg.sigma * expf(az), cfg.min_scale, cfg.max_scale);
            o[3] = clampf_(cfg.opacity_scale * expf(ol), cfg.min_opacity, cfg.max_opacity);
        } break;
    }
    reinterpret_cast<float4*>(pv)[idx] = make_float4(p.x, p.y, p.z, 1.0f);
    reinterpret_cast<float4*>(rot)[idx] = make_float4(q[0], q[1], q[2], q[3]);
    reinterpret_cast<float4*>(so)[idx] = make_float4(o[0], o[1], o[2], o[3]);
}

hipError_t launch_decode_gaussians(const float4* pos, const float* states, uint32_t count, uint32_t S,
                                   const npa_gaussian_decode_cfg& cfg, float* pv, float* sh, float* rot,
                                   float* so, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    const uint32_t K = cfg.mode == NPA_DECODE_SH0_ORIENTED ? (cfg.sh_degree + 1) * (cfg.sh_degree + 1) : 1;
    hipLaunchKernelGGL(k_decode, dim3((count + 255) / 256), dim3(256), 0, stream, pos, states, count, S, cfg, K,
                       pv, sh, rot, so);
    return hipGetLastError();
}

// ------------------------------------------------------------ viewer export
// write_gaussian_from_output  crates/burn_automata/src/gpu_step.wgsl:4963-5052 (write_gaussian_main
// 4929-4936): position (z = 0 in 2D) and visibility 1; 48 SH coefficients, zero but for the DC
// triple (clamp(tail + 0.5) - 0.5) / SH_C0 of the last three state channels (4981-4990); identity
// rotation and isotropic scale max(eps * 0.12, 8e-5), or for 3D position-feature models with
// S >= 9 the rotation taking +z onto the normal in channels 4..6 and a flattened tangent-plane
// scale (4992-5045); opacity 1 in 2D, clamp(sigmoid(channel 8, or 3 when S <= 8), 0.001, 0.95) in
// 3D (5046-5051). normalize() is v / sqrt(sum v^2) and length() sqrt(x^2 + y^2 + z^2), in that
// order (the oracle's restatement evaluates the same operations). The material branch belongs to
// the adaptive rollouts and is not built.
constexpr float kShC0 = 0.28209479177387814f;  // SH_C0 gpu_step.wgsl:7
constexpr uint32_t kShCoeffs = NPA_GAUSSIAN_SH_COEFF_COUNT;

struct ExportParams {
    uint32_t total, N, S, dim;
    float eps;
    uint32_t normal_branch;
};

__device__ __forceinline__ float export_channel(const float* s, uint32_t S, uint32_t c) {  // output_state_channel
    return c < S ? s[c] : (S > 0 ? s[0] : 0.0f);
}

// One thread per particle for the 4-float records; each wave then writes its 64 particles' SH
// rows (12 float4 each) as consecutive float4s, lane l taking float4 j * 64 + l of the wave's
// block and the DC triple from the particle's lane.
__global__ __launch_bounds__(256) void k_write_gaussians(ExportParams P, const float4* __restrict__ pos,
                                                         const float* __restrict__ states, float4* __restrict__ pv,
                                                         float4* __restrict__ sh, float4* __restrict__ rot,
                                                         float4* __restrict__ so) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    float dc[3] = {0.0f, 0.0f, 0.0f};
    if (idx < P.total) {
        const uint32_t S = P.S;
        const float* s = states + (uint64_t)idx * S;
        const float4 p = pos[idx];
        pv[idx] = make_float4(p.x, p.y, P.dim == 3 ? p.z : 0.0f, 1.0f);
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {  // output_tail_state_channel(idx, 2 - ch)
            const uint32_t off = 2u - (uint32_t)ch;
            const float tail = S > off ? export_channel(s, S, S - 1 - off) : export_channel(s, S, 0);
            const float color = clampf_(tail + 0.5f, 0.0f, 1.0f);
            dc[ch] = (color - 0.5f) / kShC0;
        }
        const float iso = fmaxf(P.eps * 0.12f, 0.00008f);
        float sc[3] = {iso, iso, iso};
        float q[4] = {1.0f, 0.0f, 0.0f, 0.0f};
        if (P.normal_branch) {
            const float n0 = export_channel(s, S, 4), n1 = export_channel(s, S, 5), n2 = export_channel(s, S, 6);
            const float nn = sqrtf(n0 * n0 + n1 * n1 + n2 * n2);
            float u0 = 0.0f, u1 = 0.0f, u2 = 1.0f;
            if (nn > 1.0e-6f && nn < 1.0e20f) {
                u0 = n0 / nn;
                u1 = n1 / nn;
                u2 = n2 / nn;
            }
            if (u2 <= -0.999999f) {
                q[0] = 0.0f;
                q[1] = 1.0f;
                q[2] = 0.0f;
                q[3] = 0.0f;
            } else {
                const float r[4] = {1.0f + u2, -u1, u0, 0.0f};
                const float rl = sqrtf(r[0] * r[0] + r[1] * r[1] + r[2] * r[2] + r[3] * r[3]);
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = r[k] / rl;
            }
            const float density_scale = clampf_(sqrtf(4096.0f / fmaxf((float)P.N, 1.0f)), 0.4f, 2.0f);
            const float tangent =
                fmaxf(clampf_(P.eps * 0.32f * density_scale, P.eps * 0.08f, P.eps * 0.64f), 0.00008f);
            sc[0] = tangent;
            sc[1] = tangent;
            sc[2] = fmaxf(tangent * 0.18f, 0.00008f);
        }
        float opacity = 1.0f;
        if (P.dim == 3) {
            const float logit = export_channel(s, S, S > 8 ? 8u : 3u);
            opacity = clampf_(1.0f / (1.0f + expf(-logit)), 0.001f, 0.95f);
        }
        rot[idx] = make_float4(q[0], q[1], q[2], q[3]);
        so[idx] = make_float4(sc[0], sc[1], sc[2], opacity * 1.0f);
    }
    constexpr uint32_t kRow = kShCoeffs / 4;  // float4s per particle
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t first = idx - lane;  // the wave's first particle
#pragma unroll
    for (uint32_t j = 0; j < kRow; ++j) {
        const uint32_t v = j * 64 + lane;
        const uint32_t pl = v / kRow, comp = v - pl * kRow;
        const float d0 = __shfl(dc[0], (int)pl, 64), d1 = __shfl(dc[1], (int)pl, 64), d2 = __shfl(dc[2], (int)pl, 64);
        if (first + pl < P.total)
            sh[(uint64_t)(first + pl) * kRow + comp] = comp == 0 ? make_float4(d0, d1, d2, 0.0f) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

hipError_t launch_write_gaussians(const float4* pos, const float* states, uint32_t total, uint32_t particle_count,
                                  uint32_t S, uint32_t dim, float eps, bool position_features, float* pv, float* sh,
                                  float* rot, float* so, hipStream_t stream) {
    if (total == 0) return hipSuccess;
    ExportParams P{total, particle_count, S, dim, eps, (dim == 3 && position_features && S >= 9) ? 1u : 0u};
    hipLaunchKernelGGL(k_write_gaussians, dim3((total + 255) / 256), dim3(256), 0, stream, P, pos, states,
                       (float4*)pv, (float4*)sh, (float4*)rot, (float4*)so);
    return hipGetLastError();
}

// ----------------------------------------------------------------- splat
constexpr int kTile = 16;

// A Gaussian weight exp(-d2 / (2 sigma^2)) (splat.rs:71, image.rs:61) as 2^(-d2 * k2) with
// k2 = log2(e) / (2 sigma^2) on the hardware exp2; it differs from expf of the IEEE quotient by a
// few ulps at most.
constexpr float kLog2e = 1.44269504088896340736f;
__device__ __forceinline__ float splat_weight(float d2, float k2) { return __builtin_amdgcn_exp2f(-(d2 * k2)); }

struct SplatParams {
    int size;
    int radius;
    int tiles_x, tiles_y;
    float sigma;      // pixel-space sigma after the normalize_color rescale
    float two_sig2;   // 2 * sigma * sigma
    float k2;         // log2(e) / two_sig2 (splat_weight)
    float norm_scale;
    float lo, hi;
    int normalize, y_up;
    int S;
    // Tiled layout: particle n belongs to window n / per_window; windows are laid out row-major,
    // win_cols per row, each size x size pixels with tiles_x * tiles_y screen tiles; the image row
    // stride is stride pixels. A single image is one window.
    uint32_t per_window, win_cols, tiles_per_win;
    int stride;
};

struct SplatParticle {  // 32 bytes
    float fx, fy;
    int bx, by;
    float scale;  // norm_scale / the normaliser (1 without normalize_color)
    float c[3];
};

__device__ __forceinline__ bool splat_tiles(const SplatParams& P, int64_t bx, int64_t by, int* tx0, int* tx1,
                                            int* ty0, int* ty1) {
    int64_t x0 = bx - P.radius, x1 = bx + P.radius, y0 = by - P.radius, y1 = by + P.radius;
    if (x0 < 0) x0 = 0;
    if (y0 < 0) y0 = 0;
    if (x1 > P.size - 1) x1 = P.size - 1;
    if (y1 > P.size - 1) y1 = P.size - 1;
    if (x0 > x1 || y0 > y1) return false;
    *tx0 = (int)(x0 / kTile);
    *tx1 = (int)(x1 / kTile);
    *ty0 = (int)(y0 / kTile);
    *ty1 = (int)(y1 / kTile);
    return true;
}

// Value of lane J of each group of four consecutive lanes (DPP quad_perm; every lane reads a valid
// lane, so bound_ctrl never applies and the compiler folds the move into the consuming add).
template <int J>
__device__ __forceinline__ float quad_bcast(float v) {
    constexpr int c = J | (J << 2) | (J << 4) | (J << 6);
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), c, 0xf, 0xf, true));
}

// Four lanes per particle: every lane derives the particle's pixel-space centre; lane q computes the
// window weights of offsets q, q + 4, ... (row-major over (oy, ox), the reference's order), and
// every lane adds each round's four weights in offset order, so the sum is the serial sum of the
// reference (an out-of-image offset adds +0.0, which leaves the non-negative sum unchanged).
__global__ __launch_bounds__(256) void k_splat_prep(SplatParams P, const float4* __restrict__ pos,
                                                    const float* __restrict__ colors,
                                                    const float* __restrict__ states, uint32_t count,
                                                    SplatParticle* __restrict__ out,
                                                    uint32_t* __restrict__ ntiles) {
    const uint32_t gt = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t q = gt & 3u;
    const uint32_t n = gt >> 2;
    const bool valid = n < count;
    const float4 p = pos[valid ? n : 0u];
    const float fsz = (float)P.size;
    const float px = (p.x - P.lo) / (P.hi - P.lo) * (fsz - 1.0f);
    float py = (p.y - P.lo) / (P.hi - P.lo) * (fsz - 1.0f);
    if (P.y_up) py = (fsz - 1.0f) - py;
    const int64_t bx = f32_to_isize(floorf(px)), by = f32_to_isize(floorf(py));
    const float fx = px - (float)bx, fy = py - (float)by;
    int tx0, tx1, ty0, ty1;
    const bool any = valid && splat_tiles(P, bx, by, &tx0, &tx1, &ty0, &ty1);
    float weight_sum = 0.0f;
    if (__ballot(any)) {
        const int side = 2 * P.radius + 1;
        const uint32_t terms = (uint32_t)side * (uint32_t)side;
        int oy = -P.radius, ox = -P.radius + (int)q;  // offset q of the row-major window
        while (ox > P.radius) {
            ox -= side;
            ++oy;
        }
        for (uint32_t k0 = 0; k0 < terms; k0 += 4) {
            float wk = 0.0f;
            const int64_t x = bx + ox, y = by + oy;
            if (any && k0 + q < terms && x >= 0 && y >= 0 && x < P.size && y < P.size) {
                const float dx = (float)ox - fx, dy = (float)oy - fy;
                wk = splat_weight(dx * dx + dy * dy, P.k2);
            }
            weight_sum += quad_bcast<0>(wk);
            weight_sum += quad_bcast<1>(wk);
            weight_sum += quad_bcast<2>(wk);
            weight_sum += quad_bcast<3>(wk);
            ox += 4;  // the offset four places on
            while (ox > P.radius) {
                ox -= side;
                ++oy;
            }
        }
    }
    if (!valid || q != 0) return;
    SplatParticle sp;
    sp.fx = fx;
    sp.fy = fy;
    sp.bx = any ? (int)bx : 0;
    sp.by = any ? (int)by : 0;
    sp.scale = P.norm_scale / (P.normalize ? fmaxf(weight_sum, 1e-8f) : 1.0f);
    if (colors) {
        sp.c[0] = colors[3 * (uint64_t)n];
        sp.c[1] = colors[3 * (uint64_t)n + 1];
        sp.c[2] = colors[3 * (uint64_t)n + 2];
    } else {  // infer_2d.rs:20-31
        const float* s = states + (uint64_t)n * P.S + (P.S - 3);
        for (int k = 0; k < 3; ++k) sp.c[k] = clampf_(s[k] + 0.5f, 0.0f, 1.0f);
    }
    out[n] = sp;
    ntiles[n] = any ? (uint32_t)((tx1 - tx0 + 1) * (ty1 - ty0 + 1)) : 0u;
}

__global__ __launch_bounds__(1024) void k_scan_1block(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                      uint32_t count, uint32_t* __restrict__ total_out) {
    __shared__ uint32_t lds[32];
    const uint32_t per = (count + blockDim.x - 1) / blockDim.x;
    const uint32_t k0 = threadIdx.x * per;
    const uint32_t k1 = k0 + per < count ? k0 + per : count;
    uint32_t sum = 0;
    // batches of 8 independent loads (one memory round trip per batch, not per element)
    for (uint32_t k = k0; k < k1; k += 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = k + u < k1 ? in[k + u] : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += v[u];
    }
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t x = sum;
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t y = __shfl_up(x, off, 64);
        if (lane >= (uint32_t)off) x += y;
    }
    if (lane == 63) lds[wid] = x;
    __syncthreads();
    if (wid == 0) {
        uint32_t s = lane < nw ? lds[lane] : 0;
        for (int off = 1; off < 64; off <<= 1) {
            uint32_t y = __shfl_up(s, off, 64);
            if (lane >= (uint32_t)off) s += y;
        }
        if (lane < nw) lds[lane] = s;
    }
    __syncthreads();
    uint32_t run = (wid ? lds[wid - 1] : 0) + x - sum;
    for (uint32_t k = k0; k < k1; k += 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = k + u < k1 ? in[k + u] : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (k + u < k1) out[k + u] = run;
            run += v[u];
        }
    }
    if (threadIdx.x == 0) *total_out = lds[nw - 1];
}

// Multi-block exclusive scan: blocks of 256 threads own 1024 consecutive values each, loaded
// coalesced through LDS; each thread scans 4 consecutive values.
constexpr uint32_t kScanBlock = 1024;

__device__ __forceinline__ uint32_t block_exclusive_256(uint32_t v, uint32_t* lds8, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= (uint32_t)off) x += y;
    }
    if (lane == 63) lds8[wid] = x;
    __syncthreads();
    uint32_t pre = 0, all = 0;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
        const uint32_t t = lds8[w];
        if (w < wid) pre += t;
        all += t;
    }
    *total = all;
    return pre + x - v;
}

__global__ __launch_bounds__(256) void k_scan_partials(const uint32_t* __restrict__ in, uint32_t count,
                                                       uint32_t* __restrict__ sums) {
    __shared__ uint32_t lds8[4];
    const uint32_t base = blockIdx.x * kScanBlock;
    uint32_t v = 0;
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
        const uint32_t k = base + u * 256 + threadIdx.x;
        v += k < count ? in[k] : 0u;
    }
    uint32_t total;
    (void)block_exclusive_256(v, lds8, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void k_scan_apply(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                    uint32_t count, const uint32_t* __restrict__ offsets) {
    __shared__ uint32_t vals[kScanBlock];
    __shared__ uint32_t lds8[4];
    const uint32_t base = blockIdx.x * kScanBlock;
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
        const uint32_t k = base + u * 256 + threadIdx.x;
        vals[u * 256 + threadIdx.x] = k < count ? in[k] : 0u;
    }
    __syncthreads();
    const uint32_t a = vals[4 * threadIdx.x], b = vals[4 * threadIdx.x + 1];
    const uint32_t c = vals[4 * threadIdx.x + 2], d = vals[4 * threadIdx.x + 3];
    uint32_t total;
    const uint32_t pre = offsets[blockIdx.x] + block_exclusive_256(a + b + c + d, lds8, &total);
    __syncthreads();
    vals[4 * threadIdx.x] = pre;
    vals[4 * threadIdx.x + 1] = pre + a;
    vals[4 * threadIdx.x + 2] = pre + a + b;
    vals[4 * threadIdx.x + 3] = pre + a + b + c;
    __syncthreads();
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
        const uint32_t k = base + u * 256 + threadIdx.x;
        if (k < count) out[k] = vals[u * 256 + threadIdx.x];
    }
}

__global__ __launch_bounds__(256) void k_splat_emit(SplatParams P, const SplatParticle* __restrict__ sp,
                                                    const uint32_t* __restrict__ ntiles,
                                                    const uint32_t* __restrict__ start, uint32_t count,
                                                    uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= count || ntiles[n] == 0) return;
    int tx0, tx1, ty0, ty1;
    splat_tiles(P, sp[n].bx, sp[n].by, &tx0, &tx1, &ty0, &ty1);
    uint32_t k = start[n];
    const uint32_t win_base = (n / P.per_window) * P.tiles_per_win;
    for (int ty = ty0; ty <= ty1; ++ty)
        for (int tx = tx0; tx <= tx1; ++tx) {
            keys[k] = win_base + (uint32_t)(ty * P.tiles_x + tx);
            vals[k] = n;
            ++k;
        }
}

__global__ __launch_bounds__(256) void k_splat_tiles(SplatParams P, const SplatParticle* __restrict__ sp,
                                                     const uint32_t* __restrict__ offsets,
                                                     const uint32_t* __restrict__ sorted, float* __restrict__ image) {
    __shared__ SplatParticle buf[256];
    const uint32_t t = blockIdx.x;
    const uint32_t win = t / P.tiles_per_win, lt = t - win * P.tiles_per_win;
    const int tx = (int)(lt % P.tiles_x), ty = (int)(lt / P.tiles_x);
    const int x = tx * kTile + (int)(threadIdx.x % kTile);
    const int y = ty * kTile + (int)(threadIdx.x / kTile);
    const uint32_t beg = offsets[t], end = offsets[t + 1];
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t base = beg; base < end; base += 256) {
        const uint32_t k = base + threadIdx.x;
        if (k < end) buf[threadIdx.x] = sp[sorted[k]];
        __syncthreads();
        const uint32_t m = end - base < 256 ? end - base : 256;
        for (uint32_t q = 0; q < m; ++q) {
            const SplatParticle& p = buf[q];
            const int ox = x - p.bx, oy = y - p.by;
            if (ox < -P.radius || ox > P.radius || oy < -P.radius || oy > P.radius) continue;
            const float dx = (float)ox - p.fx, dy = (float)oy - p.fy;
            const float w = splat_weight(dx * dx + dy * dy, P.k2) * p.scale;
            acc[0] += p.c[0] * w;
            acc[1] += p.c[1] * w;
            acc[2] += p.c[2] * w;
            acc[3] += w;
        }
        __syncthreads();
    }
    if (x < P.size && y < P.size) {
        const uint64_t row = (uint64_t)(win / P.win_cols) * P.size + y;
        const uint64_t col = (uint64_t)(win % P.win_cols) * P.size + x;
        reinterpret_cast<float4*>(image)[row * P.stride + col] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
}

void SplatWorkspace::release() {
    for (DevBuf* b : {&params, &item_start, &keys, &vals, &sorted, &ranks, &table, &totals, &offsets, &count, &flags, &scan,
                      &attrs, &partials, &chunks, &order, &decoded, &sort_temp})
        b->release();
}

hipError_t launch_splat_2d(const float4* pos, const float* colors, const float* states, uint32_t S,
                           uint32_t count, const npa_splat2d_cfg& cfg, float* image, SplatWorkspace& ws,
                           hipStream_t stream, Profiler* prof, uint32_t per_window, uint32_t windows,
                           uint32_t win_cols) {
    SplatParams P{};
    P.size = (int)cfg.image_size;
    const float fsz = (float)cfg.image_size;
    float sigma = cfg.sigma;  // splat.rs:36-46
    if (cfg.normalize_color) sigma = sigma * fsz * cfg.pixel_size / (cfg.hi - cfg.lo);
    float rf = ceilf(5.0f * sigma);
    if (!(rf >= 1.0f)) rf = rf != rf ? 1.0f : 1.0f;
    if (rf > 4096.0f) rf = 4096.0f;  // windows wider than any supported image are clipped anyway
    P.radius = (int)rf;
    P.sigma = sigma;
    P.two_sig2 = 2.0f * sigma * sigma;
    P.k2 = kLog2e / P.two_sig2;
    P.norm_scale = 1.0f;
    if (cfg.normalize_color) {
        const float t = fsz * cfg.pixel_size / (cfg.hi - cfg.lo);
        P.norm_scale = t * t;
    }
    P.lo = cfg.lo;
    P.hi = cfg.hi;
    P.normalize = cfg.normalize_color ? 1 : 0;
    P.y_up = cfg.y_up ? 1 : 0;
    P.S = (int)S;
    P.tiles_x = (P.size + kTile - 1) / kTile;
    P.tiles_y = P.tiles_x;
    if (windows == 0 || win_cols == 0 || per_window == 0) return hipErrorInvalidValue;
    if ((uint64_t)per_window * windows < count) return hipErrorInvalidValue;
    P.per_window = per_window;
    P.win_cols = win_cols;
    P.tiles_per_win = (uint32_t)(P.tiles_x * P.tiles_y);
    P.stride = (int)(win_cols * (uint32_t)P.size);
    const uint64_t ntile64 = (uint64_t)P.tiles_per_win * windows;
    if (ntile64 > 65536) return hipErrorInvalidValue;  // the key sort's bin limit
    const uint32_t ntile_total = (uint32_t)ntile64;
    const uint32_t ntile_win = P.tiles_per_win;
    const uint64_t per_axis = (uint64_t)((2 * P.radius + 1 + kTile - 1) / kTile + 1);
    const uint64_t max_per = std::min<uint64_t>(per_axis * per_axis, ntile_win);
    const uint64_t cap64 = (uint64_t)count * max_per;
    if (cap64 >= (1ull << 31)) return hipErrorInvalidValue;
    const uint32_t cap = (uint32_t)cap64;
    HashgridPlan plan;
    if (!make_key_sort_plan(cap, ntile_total, &plan)) return hipErrorInvalidValue;
    hipError_t e;
#define NPA_RES(buf, n) \
    if ((e = (buf).reserve((size_t)(n))) != hipSuccess) return e;
    NPA_RES(ws.params, (uint64_t)(count ? count : 1) * sizeof(SplatParticle));
    NPA_RES(ws.item_start, (uint64_t)(count ? count : 1) * 8);
    NPA_RES(ws.keys, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.vals, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.sorted, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.ranks, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.table, plan.table_entries * 4);
    NPA_RES(ws.totals, (uint64_t)ntile_total * 4);
    NPA_RES(ws.offsets, ((uint64_t)ntile_total + 1) * 4);
    NPA_RES(ws.count, 64);
    NPA_RES(ws.scan, (2 * ((uint64_t)count / kScanBlock + 1) + 2) * 4);
    NPA_RES(ws.flags, 64);
#undef NPA_RES
    ProfScope ps(prof, NPA_KERNEL_SPLAT, stream);
    uint32_t* ntiles = ws.item_start.as<uint32_t>() + (count ? count : 1);
    uint32_t* start = ws.item_start.as<uint32_t>();
    if (count) {
        hipLaunchKernelGGL(k_splat_prep, dim3((uint32_t)(((uint64_t)count * 4 + 255) / 256)), dim3(256), 0, stream, P,
                           pos, colors, states, count, ws.params.as<SplatParticle>(), ntiles);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    {  // start = exclusive prefix of ntiles, total item count into ws.count
        const uint32_t nb = (count + kScanBlock - 1) / kScanBlock;
        uint32_t* sums = ws.scan.as<uint32_t>();
        if (nb) {
            hipLaunchKernelGGL(k_scan_partials, dim3(nb), dim3(256), 0, stream, ntiles, count, sums);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k_scan_1block, dim3(1), dim3(1024), 0, stream, sums, sums + nb + 1, nb,
                           ws.count.as<uint32_t>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (nb) {
            hipLaunchKernelGGL(k_scan_apply, dim3(nb), dim3(256), 0, stream, ntiles, start, count, sums + nb + 1);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    if (count) {
        hipLaunchKernelGGL(k_splat_emit, dim3((count + 255) / 256), dim3(256), 0, stream, P,
                           ws.params.as<SplatParticle>(), ntiles, start, count, ws.keys.as<uint32_t>(),
                           ws.vals.as<uint32_t>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    e = launch_key_sort(plan, ws.keys.as<uint32_t>(), ws.vals.as<uint32_t>(), ws.count.as<uint32_t>(), cap,
                        ws.ranks.as<uint32_t>(), ws.table.as<uint32_t>(), ws.totals.as<uint32_t>(),
                        ws.offsets.as<uint32_t>(), ws.sorted.as<uint32_t>(), ws.flags.as<uint32_t>(), stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_splat_tiles, dim3(ntile_total), dim3(256), 0, stream, P, ws.params.as<SplatParticle>(),
                       ws.offsets.as<uint32_t>(), ws.sorted.as<uint32_t>(), image);
    return hipGetLastError();
}

// ------------------------------------------------------- projected 3D render
// project_positions (render_loss/projection.rs:11-29) + splat_projected (render_loss/image.rs:18-79)
// for up to kMaxRenderViews views in one pipeline: item i = v * count + n is particle n seen
// through view v; its screen tiles get keys v * tiles_per_view + tile, so one stable key sort
// bins every view, and one tile kernel draws them all. Within a tile the items keep ascending
// n, so every pixel sums its particles in the reference's order.
constexpr float kRenderEps = 1.0e-8f;

struct RenderParams {
    int size, tiles_x;
    uint32_t tiles_per_view, count;
    float ws, min_sigma, max_sigma, norm_scale;
    float basis[kMaxRenderViews][9];  // right, up, forward of each view
};

struct alignas(16) RenderParticle {  // 48 bytes
    float px, py;     // projected pixel coordinates
    int x0, y0;       // first column / row of the (2 radius + 1)^2 footprint (image.rs:41-53)
    uint32_t span;    // 2 radius
    float k2;         // log2(e) / (2 sigma^2)
    float scale;      // norm_scale * clamp(opacity, 0, 1) / max(in-bounds weight sum, EPS)
    float depth;
    float c[3];
    float pad;
};


__device__ __forceinline__ bool render_tiles(const RenderParams& P, int64_t bx, int64_t by, int64_t r, int* tx0,
                                             int* tx1, int* ty0, int* ty1) {
    int64_t x0 = bx - r, x1 = bx + r, y0 = by - r, y1 = by + r;
    if (x0 < 0) x0 = 0;
    if (y0 < 0) y0 = 0;
    if (x1 > P.size - 1) x1 = P.size - 1;
    if (y1 > P.size - 1) y1 = P.size - 1;
    if (x0 > x1 || y0 > y1) return false;
    *tx0 = (int)(x0 / kTile);
    *tx1 = (int)(x1 / kTile);
    *ty0 = (int)(y0 / kTile);
    *ty1 = (int)(y1 / kTile);
    return true;
}

// kPrepLanes lanes per particle-view; grid (ceil(count * kPrepLanes / 256), nviews): blockIdx.y is
// the view, so its basis is a uniform load. The lanes split the in-bounds footprint by rows (lane
// l sums rows l, l + kPrepLanes, ... left to right) and combine their sums in a fixed butterfly,
// so the weight sum is deterministic; it differs from the reference's single running sum only
// by rounding.
constexpr uint32_t kPrepLanes = 16;

__global__ __launch_bounds__(256) void k_render_prep(RenderParams P, const float4* __restrict__ pos,
                                                     const float* __restrict__ colors,
                                                     const float* __restrict__ opacities,
                                                     const float* __restrict__ sigmas,
                                                     RenderParticle* __restrict__ out,
                                                     uint32_t* __restrict__ ntiles) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t n = g / kPrepLanes, lane = g % kPrepLanes;
    const bool live = n < P.count;  // the whole group agrees: count * kPrepLanes threads are live
    const uint32_t nn = live ? n : 0;
    const uint32_t v = blockIdx.y;
    const float* B = P.basis[v];
    const float4 p = pos[nn];
    // dot3 (math.rs:20-22) in the reference's order, then the depth of projection.rs:20-21
    const float x = p.x * B[0] + p.y * B[1] + p.z * B[2];
    const float y = p.x * B[3] + p.y * B[4] + p.z * B[5];
    const float f = p.x * B[6] + p.y * B[7] + p.z * B[8];
    const float depth = clampf_(0.5f + 0.5f * f / fmaxf(P.ws, kRenderEps), 0.0f, 1.0f);
    const float sigma = fmaxf(clampf_(sigmas[nn], P.min_sigma, P.max_sigma), kRenderEps);
    const float sigma2 = sigma * sigma;
    const float k2 = kLog2e / (2.0f * sigma2);
    const int64_t radius = f32_to_isize(fmaxf(ceilf(5.0f * sigma), 1.0f));
    const float fsz1 = (float)P.size - 1.0f;
    const float px = (x + P.ws) / (2.0f * P.ws) * fsz1;
    const float py = (P.ws - y) / (2.0f * P.ws) * fsz1;
    const int64_t bx = f32_to_isize(floorf(px)), by = f32_to_isize(floorf(py));
    const float fx = px - (float)bx, fy = py - (float)by;
    int tx0 = 0, tx1 = -1, ty0 = 0, ty1 = -1;
    const bool any = live && render_tiles(P, bx, by, radius, &tx0, &tx1, &ty0, &ty1);
    float part = 0.0f;
    if (any) {  // the in-bounds part of the footprint (image.rs:49-63)
        const int oy0 = (int)(by - radius < 0 ? -by : -radius);
        const int oy1 = (int)(by + radius > P.size - 1 ? P.size - 1 - by : radius);
        const int ox0 = (int)(bx - radius < 0 ? -bx : -radius);
        const int ox1 = (int)(bx + radius > P.size - 1 ? P.size - 1 - bx : radius);
        for (int oy = oy0 + (int)lane; oy <= oy1; oy += (int)kPrepLanes) {
            const float dy = (float)oy - fy;
            for (int ox = ox0; ox <= ox1; ++ox) {
                const float dx = (float)ox - fx;
                part += splat_weight(dx * dx + dy * dy, k2);
            }
        }
    }
#pragma unroll
    for (uint32_t m = kPrepLanes / 2; m >= 1; m >>= 1) part += __shfl_xor(part, (int)m, (int)kPrepLanes);
    if (!live || lane != 0) return;
    const uint64_t i = (uint64_t)v * P.count + n;
    RenderParticle rp;
    rp.px = px;
    rp.py = py;
    rp.x0 = any ? (int)(bx - radius) : 0;
    rp.y0 = any ? (int)(by - radius) : 0;
    rp.span = any ? (uint32_t)(2 * radius) : 0u;
    rp.k2 = k2;
    rp.scale = P.norm_scale * clampf_(opacities[n], 0.0f, 1.0f) / fmaxf(part, kRenderEps);  // image.rs:67-69
    rp.depth = depth;
    rp.c[0] = colors[3 * (uint64_t)n];
    rp.c[1] = colors[3 * (uint64_t)n + 1];
    rp.c[2] = colors[3 * (uint64_t)n + 2];
    rp.pad = 0.0f;
    out[i] = rp;
    ntiles[i] = any ? (uint32_t)((tx1 - tx0 + 1) * (ty1 - ty0 + 1)) : 0u;
}

__global__ __launch_bounds__(256) void k_render_emit(RenderParams P, const RenderParticle* __restrict__ rp,
                                                     const uint32_t* __restrict__ ntiles,
                                                     const uint32_t* __restrict__ start, uint32_t items,
                                                     uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= items || ntiles[i] == 0) return;
    const RenderParticle q = rp[i];
    const int64_t r = q.span / 2;
    int tx0, tx1, ty0, ty1;
    render_tiles(P, (int64_t)q.x0 + r, (int64_t)q.y0 + r, r, &tx0, &tx1, &ty0, &ty1);
    uint32_t k = start[i];
    const uint32_t base = (i / P.count) * P.tiles_per_view;
    for (int ty = ty0; ty <= ty1; ++ty)
        for (int tx = tx0; tx <= tx1; ++tx) {
            keys[k] = base + (uint32_t)(ty * P.tiles_x + tx);
            vals[k] = i;
            ++k;
        }
}

// The sorted particle list of each screen tile is cut into chunks of kChunk particles; a block
// draws one chunk of one tile (thread = pixel, the chunk staged in LDS), summing its particles in
// ascending index order into a partial tile. k_render_reduce then adds each tile's partials in
// chunk order. A tile of one chunk is thus exactly the reference's running sum; a longer list
// differs from it only by the rounding of the chunk boundaries.
constexpr uint32_t kChunk = 256;

// One block: nch[t] = ceil(tile t's key count / kChunk), chunk_start = its exclusive prefix, and
// the total into *total. ntiles <= 65536, so each thread owns at most 64 consecutive tiles.
__global__ __launch_bounds__(1024) void k_render_chunk_scan(const uint32_t* __restrict__ offsets, uint32_t ntiles,
                                                            uint32_t* __restrict__ nch,
                                                            uint32_t* __restrict__ chunk_start,
                                                            uint32_t* __restrict__ total) {
    __shared__ uint32_t lds[16];
    const uint32_t per = (ntiles + blockDim.x - 1) / blockDim.x;
    const uint32_t t0 = threadIdx.x * per;
    const uint32_t t1 = t0 + per < ntiles ? t0 + per : ntiles;
    uint32_t sum = 0;
    for (uint32_t t = t0; t < t1; ++t) {
        const uint32_t c = (offsets[t + 1] - offsets[t] + kChunk - 1) / kChunk;
        nch[t] = c;
        sum += c;
    }
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t x = sum;
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= (uint32_t)off) x += y;
    }
    if (lane == 63) lds[wid] = x;
    __syncthreads();
    uint32_t base = 0, all = 0;
    for (uint32_t w = 0; w < nw; ++w) {
        const uint32_t v = lds[w];
        if (w < wid) base += v;
        all += v;
    }
    uint32_t run = base + x - sum;
    for (uint32_t t = t0; t < t1; ++t) {
        chunk_start[t] = run;
        run += nch[t];
    }
    if (threadIdx.x == 0) *total = all;
}

// Grid-stride over the chunks; thread = pixel, the chunk's particles staged in LDS. dx = x - px
// is the reference's (x - base_x) - frac_x exactly: both are one rounding of the same real number.
// partials[c][5][256] (channel-planar, so the stores coalesce).
__global__ __launch_bounds__(256) void k_render_chunks(RenderParams P, const RenderParticle* __restrict__ rp,
                                                       const uint32_t* __restrict__ offsets,
                                                       const uint32_t* __restrict__ sorted,
                                                       const uint32_t* __restrict__ chunk_start,
                                                       const uint32_t* __restrict__ total_chunks, uint32_t ntiles,
                                                       float* __restrict__ partials) {
    __shared__ RenderParticle buf[kChunk];
    const uint32_t total = *total_chunks;
    for (uint32_t c = blockIdx.x; c < total; c += gridDim.x) {
        // the tile: the last t with chunk_start[t] <= c (tiles without chunks share the next start)
        uint32_t lo = 0, hi = ntiles - 1;
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) / 2;
            if (chunk_start[mid] <= c) lo = mid;
            else hi = mid - 1;
        }
        const uint32_t t = lo;
        const uint32_t v = t / P.tiles_per_view, lt = t - v * P.tiles_per_view;
        const int x = (int)(lt % (uint32_t)P.tiles_x) * kTile + (int)(threadIdx.x % kTile);
        const int y = (int)(lt / (uint32_t)P.tiles_x) * kTile + (int)(threadIdx.x / kTile);
        const float xf = (float)x, yf = (float)y;
        const uint32_t beg = offsets[t] + (c - chunk_start[t]) * kChunk;
        const uint32_t end = min(beg + kChunk, offsets[t + 1]);
        if (beg + threadIdx.x < end) buf[threadIdx.x] = rp[sorted[beg + threadIdx.x]];
        __syncthreads();
        float acc[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t m = end - beg;
        for (uint32_t q = 0; q < m; ++q) {
            const RenderParticle& p = buf[q];
            if ((uint32_t)(x - p.x0) > p.span || (uint32_t)(y - p.y0) > p.span) continue;
            const float dx = xf - p.px, dy = yf - p.py;
            const float w = splat_weight(dx * dx + dy * dy, p.k2) * p.scale;  // image.rs:61, 69
            acc[0] += p.c[0] * w;
            acc[1] += p.c[1] * w;
            acc[2] += p.c[2] * w;
            acc[3] += w;
            acc[4] += p.depth * w;
        }
        float* o = partials + (uint64_t)c * (5 * kChunk) + threadIdx.x;
#pragma unroll
        for (int ch = 0; ch < 5; ++ch) o[ch * kChunk] = acc[ch];
        __syncthreads();  // buf is refilled by the next chunk
    }
}

// One tile per block, thread = pixel: the tile's partials in chunk order (zero for an empty tile).
__global__ __launch_bounds__(256) void k_render_reduce(RenderParams P, const uint32_t* __restrict__ chunk_start,
                                                       const uint32_t* __restrict__ nch,
                                                       const float* __restrict__ partials,
                                                       float* __restrict__ images) {
    const uint32_t t = blockIdx.x;
    const uint32_t v = t / P.tiles_per_view, lt = t - v * P.tiles_per_view;
    const int x = (int)(lt % (uint32_t)P.tiles_x) * kTile + (int)(threadIdx.x % kTile);
    const int y = (int)(lt / (uint32_t)P.tiles_x) * kTile + (int)(threadIdx.x / kTile);
    float acc[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t c0 = chunk_start[t], c1 = c0 + nch[t];
    uint32_t c = c0;
    for (; c + 4 <= c1; c += 4) {  // four chunks' loads in flight, then added in chunk order
        float v[4][5];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float* q = partials + (uint64_t)(c + u) * (5 * kChunk) + threadIdx.x;
#pragma unroll
            for (int ch = 0; ch < 5; ++ch) v[u][ch] = q[ch * kChunk];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int ch = 0; ch < 5; ++ch) acc[ch] += v[u][ch];
    }
    for (; c < c1; ++c) {
        const float* q = partials + (uint64_t)c * (5 * kChunk) + threadIdx.x;
#pragma unroll
        for (int ch = 0; ch < 5; ++ch) acc[ch] += q[ch * kChunk];
    }
    if (x < P.size && y < P.size) {
        float* o = images + (((uint64_t)v * P.size + y) * P.size + x) * 5;
#pragma unroll
        for (int ch = 0; ch < 5; ++ch) o[ch] = acc[ch];
    }
}

// view_basis (render_loss/projection.rs:31-43) with normalize3 / cross3 (render_loss/math.rs:24-39).
static void render_normalize3(const float v[3], float* out) {
    const float norm = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    if (norm <= kRenderEps) {
        out[0] = 0.0f;
        out[1] = 0.0f;
        out[2] = 1.0f;
        return;
    }
    for (int k = 0; k < 3; ++k) out[k] = v[k] / norm;
}

static bool render_view_basis(uint32_t view, float* b /* right, up, forward */) {
    static const int axes[3][3] = {{0, 1, 2}, {0, 2, 1}, {1, 2, 0}};  // Xy, Xz, Yz
    if (view < 3) {
        for (int k = 0; k < 9; ++k) b[k] = 0.0f;
        for (int r = 0; r < 3; ++r) b[3 * r + axes[view][r]] = 1.0f;
        return true;
    }
    if (view != NPA_VIEW_ISO) return false;
    const float a[3] = {1.0f, -1.0f, 0.0f}, u[3] = {1.0f, 1.0f, 2.0f};
    render_normalize3(a, b);
    render_normalize3(u, b + 3);
    const float* r = b;
    const float* up = b + 3;
    const float c[3] = {r[1] * up[2] - r[2] * up[1], r[2] * up[0] - r[0] * up[2], r[0] * up[1] - r[1] * up[0]};
    render_normalize3(c, b + 6);
    return true;
}

hipError_t launch_render_views(const float4* pos, const float* colors, const float* opacities, const float* sigmas,
                               uint32_t count, const uint32_t* views, uint32_t nviews, const npa_render_cfg& cfg,
                               float* images, SplatWorkspace& ws, hipStream_t stream, Profiler* prof) {
    if (nviews == 0 || nviews > kMaxRenderViews || !views) return hipErrorInvalidValue;
    RenderParams P{};
    P.size = (int)cfg.image_size;
    P.tiles_x = (P.size + kTile - 1) / kTile;
    P.tiles_per_view = (uint32_t)(P.tiles_x * P.tiles_x);
    P.count = count;
    P.ws = cfg.world_scale;
    P.min_sigma = cfg.min_sigma;
    P.max_sigma = cfg.max_sigma;
    P.norm_scale = 1.0f / (float)(count > 1 ? count : 1);  // image.rs:29
    for (uint32_t v = 0; v < nviews; ++v)
        if (!render_view_basis(views[v], P.basis[v])) return hipErrorInvalidValue;
    const uint64_t ntile64 = (uint64_t)P.tiles_per_view * nviews;
    if (ntile64 > 65536) return hipErrorInvalidValue;  // the key sort's bin limit
    const uint32_t ntile_total = (uint32_t)ntile64;
    const uint64_t items64 = (uint64_t)count * nviews;
    if (items64 >= (1ull << 31) || (uint64_t)count * kPrepLanes >= (1ull << 32)) return hipErrorInvalidValue;
    const uint32_t items = (uint32_t)items64;
    // the widest footprint: sigma <= max(max_sigma, EPS)
    const float rmaxf = fmaxf(ceilf(5.0f * fmaxf(cfg.max_sigma, kRenderEps)), 1.0f);
    if (!(rmaxf <= 1024.0f)) return hipErrorInvalidValue;
    const uint64_t per_axis = (uint64_t)((2 * (int)rmaxf + 1 + kTile - 1) / kTile + 1);
    const uint64_t max_per = std::min<uint64_t>(per_axis * per_axis, P.tiles_per_view);
    const uint64_t cap64 = items64 * max_per;
    if (cap64 >= (1ull << 31)) return hipErrorInvalidValue;
    const uint32_t cap = (uint32_t)cap64;
    HashgridPlan plan;
    if (!make_key_sort_plan(cap, ntile_total, &plan)) return hipErrorInvalidValue;
    hipError_t e;
#define NPA_RES(buf, n) \
    if ((e = (buf).reserve((size_t)(n))) != hipSuccess) return e;
    NPA_RES(ws.params, (uint64_t)(items ? items : 1) * sizeof(RenderParticle));
    NPA_RES(ws.item_start, (uint64_t)(items ? items : 1) * 8);
    NPA_RES(ws.keys, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.vals, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.sorted, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.ranks, (uint64_t)(cap ? cap : 1) * 4);
    NPA_RES(ws.table, plan.table_entries * 4);
    NPA_RES(ws.totals, (uint64_t)ntile_total * 4);
    NPA_RES(ws.offsets, ((uint64_t)ntile_total + 1) * 4);
    NPA_RES(ws.count, 64);
    NPA_RES(ws.scan, (2 * ((uint64_t)items / kScanBlock + 1) + 2) * 4);
    NPA_RES(ws.flags, 64);
    // chunks: at most one partial per kChunk keys plus one per tile
    const uint64_t max_chunks = (uint64_t)cap / kChunk + ntile_total;
    NPA_RES(ws.partials, max_chunks * 5 * kChunk * 4);
    NPA_RES(ws.chunks, (2 * (uint64_t)ntile_total + 1) * 4);
#undef NPA_RES
    ProfScope ps(prof, NPA_KERNEL_RENDER, stream);
    uint32_t* ntiles = ws.item_start.as<uint32_t>() + (items ? items : 1);
    uint32_t* start = ws.item_start.as<uint32_t>();
    RenderParticle* rp = ws.params.as<RenderParticle>();
    if (count) {
        hipLaunchKernelGGL(k_render_prep, dim3((uint32_t)(((uint64_t)count * kPrepLanes + 255) / 256), nviews), dim3(256),
                           0, stream, P, pos, colors,
                           opacities, sigmas, rp, ntiles);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    {  // start = exclusive prefix of ntiles, total key count into ws.count
        const uint32_t nb = (items + kScanBlock - 1) / kScanBlock;
        uint32_t* sums = ws.scan.as<uint32_t>();
        if (nb) {
            hipLaunchKernelGGL(k_scan_partials, dim3(nb), dim3(256), 0, stream, ntiles, items, sums);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k_scan_1block, dim3(1), dim3(1024), 0, stream, sums, sums + nb + 1, nb,
                           ws.count.as<uint32_t>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (nb) {
            hipLaunchKernelGGL(k_scan_apply, dim3(nb), dim3(256), 0, stream, ntiles, start, items, sums + nb + 1);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    if (items) {
        hipLaunchKernelGGL(k_render_emit, dim3((items + 255) / 256), dim3(256), 0, stream, P, rp, ntiles, start, items,
                           ws.keys.as<uint32_t>(), ws.vals.as<uint32_t>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    e = launch_key_sort(plan, ws.keys.as<uint32_t>(), ws.vals.as<uint32_t>(), ws.count.as<uint32_t>(), cap,
                        ws.ranks.as<uint32_t>(), ws.table.as<uint32_t>(), ws.totals.as<uint32_t>(),
                        ws.offsets.as<uint32_t>(), ws.sorted.as<uint32_t>(), ws.flags.as<uint32_t>(), stream);
    if (e != hipSuccess) return e;
    {  // chunks per tile, their exclusive prefix and total, then the chunks and the reduction
        uint32_t* nch = ws.chunks.as<uint32_t>();
        uint32_t* cstart = nch + ntile_total;
        uint32_t* ctotal = cstart + ntile_total;
        hipLaunchKernelGGL(k_render_chunk_scan, dim3(1), dim3(1024), 0, stream, ws.offsets.as<uint32_t>(), ntile_total,
                           nch, cstart, ctotal);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const uint32_t grid = (uint32_t)std::min<uint64_t>(max_chunks, 4096);
        hipLaunchKernelGGL(k_render_chunks, dim3(grid), dim3(256), 0, stream, P, rp, ws.offsets.as<uint32_t>(),
                           ws.sorted.as<uint32_t>(), cstart, ctotal, ntile_total, ws.partials.as<float>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(k_render_reduce, dim3(ntile_total), dim3(256), 0, stream, P, cstart, nch,
                           ws.partials.as<float>(), images);
    }
    return hipGetLastError();
}

// state_tail_render_attributes (render_loss/attributes.rs:15-87): one thread per particle.
__global__ __launch_bounds__(256) void k_render_attrs(const float* __restrict__ states, uint32_t count, uint32_t S,
                                                      npa_render_cfg cfg, float* __restrict__ colors,
                                                      float* __restrict__ opacities, float* __restrict__ sigmas,
                                                      float* __restrict__ derivatives) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float* s = states + (uint64_t)i * S;
    for (uint32_t k = 0; k < 3; ++k) colors[3 * (uint64_t)i + k] = clampf_(s[S - 3 + k] + 0.5f, 0.0f, 1.0f);
    // growth_3d_material_opacity_channel (rollout/mod.rs:37-45)
    const int ch = S > 8 ? 8 : (S > 3 ? 3 : -1);
    float opacity = 0.95f;  // RENDER_MAX_OPACITY (render_loss.rs:23)
    if (ch >= 0) {
        const float z = s[ch] + cfg.opacity_logit_bias;
        float sg;  // sigmoid (render_loss/math.rs:11-18)
        if (z >= 0.0f) {
            sg = 1.0f / (1.0f + expf(-z));
        } else {
            const float e = expf(z);
            sg = e / (1.0f + e);
        }
        opacity = clampf_(sg, 0.001f, 0.95f);
    }
    opacities[i] = opacity;
    float sigma, derivative = 0.0f;
    switch (cfg.gaussian_decode_mode) {
        case NPA_DECODE_PARTICLE_POINT: sigma = fmaxf(cfg.min_sigma, kRenderEps); break;
        case NPA_DECODE_SH0_LEARNED_SCALE: {
            const float logit = clampf_(s[S - 5], -8.0f, 8.0f);
            const float raw = cfg.sigma * expf(logit);
            sigma = clampf_(raw, cfg.min_sigma, cfg.max_sigma);
            derivative = (raw > cfg.min_sigma && raw < cfg.max_sigma) ? raw : 0.0f;
        } break;
        default: sigma = clampf_(cfg.sigma, cfg.min_sigma, cfg.max_sigma); break;
    }
    sigmas[i] = sigma;
    if (derivatives) derivatives[i] = derivative;
}

hipError_t launch_render_attributes(const float* states, uint32_t count, uint32_t S, const npa_render_cfg& cfg,
                                    float* colors, float* opacities, float* sigmas, float* derivatives,
                                    hipStream_t stream) {
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(k_render_attrs, dim3((count + 255) / 256), dim3(256), 0, stream, states, count, S, cfg, colors,
                       opacities, sigmas, derivatives);
    return hipGetLastError();
}


// ------------------------------------------------------------------ oriented Gaussian raster
// The EWA raster of the planar Gaussian export (the image the reference's viewer draws through
// the un-vendored bevy_gaussian_splatting 8.0.1, crates/bevy_automata/src/viewer/cloud.rs:80-97),
// restating the published 3D Gaussian splatting forward pass (Kerbl et al. 2023; EWA projection,
// Zwicker et al. 2001):
//   k_raster_prep      per Gaussian: camera-frame centre, cull, Sigma = R S S^T R^T, the EWA 2D
//                      covariance + 0.3 px^2, its conic, 3-sigma radius, tile rectangle, colour
//                      (spherical harmonics or RGB), the tile count and the depth key;
//   depth order        a stable radix sort of the indices by the positive depth's float bits
//                      (rocPRIM): depth ascending, ties by index;
//   k_raster_emit      the (tile, Gaussian) items in depth order, after a prefix of the tile
//                      counts (its total read back to size the item buffers);
//   stable key sort    by tile (the hashgrid's counting sort) -> per-tile lists in depth order;
//   k_raster_tiles     one 256-thread block per 16x16 tile, one pixel per thread: the list is
//                      staged through LDS 256 Gaussians at a time; each pixel composites front to
//                      back and stops at the transmittance cut; the block leaves when every pixel
//                      has stopped.
struct RasterParams {
    float view[12];
    float fx, fy, cx, cy, limx, limy, near_plane, far_plane;
    float campos[3];
    uint32_t width, height, tiles_x, tiles_y, count, K, sh_degree, color_mode;
    uint32_t stride;  // coefficient triples per Gaussian in the input (>= K)
};

struct alignas(16) RasterSplat {  // 48 bytes
    float mx, my, qa, qb;  // qa, qb, qc: the conic scaled by -log2(e)/2, -log2(e), -log2(e)/2
    float qc, opacity, r, g;
    float b;
    uint32_t rx;  // tile columns [rx & 0xffff, rx >> 16)
    uint32_t ry;  // tile rows
    uint32_t pad;
};

constexpr uint32_t kRasterMaxAxis = 16384;  // pixels per axis: tile indices fit 16 bits
constexpr uint32_t kDepthCulled = 0x7f800000u;  // +inf: sorts after every live depth

__device__ __forceinline__ float raster_clamp(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

__global__ __launch_bounds__(256) void k_raster_prep(RasterParams P, const float4* __restrict__ pv,
                                                     const float* __restrict__ sh, const float4* __restrict__ rot,
                                                     const float4* __restrict__ so, RasterSplat* __restrict__ out,
                                                     uint32_t* __restrict__ ntiles, uint32_t* __restrict__ dkey) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= P.count) return;
    ntiles[i] = 0;
    dkey[i] = kDepthCulled;
    const float4 p = pv[i];
    if (!(p.w > 0.0f)) return;
    const float* V = P.view;
    const float vx = V[0] * p.x + V[1] * p.y + V[2] * p.z + V[3];
    const float vy = V[4] * p.x + V[5] * p.y + V[6] * p.z + V[7];
    const float vz = V[8] * p.x + V[9] * p.y + V[10] * p.z + V[11];
    const float tx = vx, ty = -vy, tz = -vz;  // x right, y down, z forward
    if (!(tz > P.near_plane) || !(tz <= P.far_plane)) return;
    const float4 q4 = rot[i];
    float qw = q4.x, qx = q4.y, qy = q4.z, qz = q4.w;
    const float qn = sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
    if (qn > 0.0f && qn < INFINITY) {
        qw = qw / qn; qx = qx / qn; qy = qy / qn; qz = qz / qn;
    } else {
        qw = 1.0f; qx = qy = qz = 0.0f;
    }
    const float R[3][3] = {
        {1.0f - 2.0f * (qy * qy + qz * qz), 2.0f * (qx * qy - qw * qz), 2.0f * (qx * qz + qw * qy)},
        {2.0f * (qx * qy + qw * qz), 1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz - qw * qx)},
        {2.0f * (qx * qz - qw * qy), 2.0f * (qy * qz + qw * qx), 1.0f - 2.0f * (qx * qx + qy * qy)}};
    const float4 s4 = so[i];
    const float sc[3] = {s4.x, s4.y, s4.z};
    float M[3][3], S[3][3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) M[r][c] = R[r][c] * sc[c];
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) S[r][c] = M[r][0] * M[c][0] + M[r][1] * M[c][1] + M[r][2] * M[c][2];
    const float W[3][3] = {{V[0], V[1], V[2]}, {-V[4], -V[5], -V[6]}, {-V[8], -V[9], -V[10]}};
    const float jx = raster_clamp(tx / tz, -P.limx, P.limx) * tz;
    const float jy = raster_clamp(ty / tz, -P.limy, P.limy) * tz;
    const float J[2][3] = {{P.fx / tz, 0.0f, -(P.fx * jx) / (tz * tz)}, {0.0f, P.fy / tz, -(P.fy * jy) / (tz * tz)}};
    float T[2][3], U[2][3];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) T[r][c] = J[r][0] * W[0][c] + J[r][1] * W[1][c] + J[r][2] * W[2][c];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 3; ++c) U[r][c] = T[r][0] * S[0][c] + T[r][1] * S[1][c] + T[r][2] * S[2][c];
    const float a = (U[0][0] * T[0][0] + U[0][1] * T[0][1] + U[0][2] * T[0][2]) + 0.3f;
    const float b = U[0][0] * T[1][0] + U[0][1] * T[1][1] + U[0][2] * T[1][2];
    const float c = (U[1][0] * T[1][0] + U[1][1] * T[1][1] + U[1][2] * T[1][2]) + 0.3f;
    const float det = a * c - b * b;
    if (!(det > 0.0f) || !(det < INFINITY)) return;
    const float mid = 0.5f * (a + c);
    const float lam = mid + sqrtf(fmaxf(0.1f, mid * mid - det));
    const float radius = ceilf(3.0f * sqrtf(lam));
    const float mx = P.cx + P.fx * tx / tz;
    const float my = P.cy + P.fy * ty / tz;
    if (!(fabsf(mx) < 1e30f) || !(fabsf(my) < 1e30f) || !(radius < 1e30f)) return;
    const uint32_t x0 = (uint32_t)raster_clamp(floorf((mx - radius) / 16.0f), 0.0f, (float)P.tiles_x);
    const uint32_t x1 = (uint32_t)raster_clamp(floorf((mx + radius) / 16.0f) + 1.0f, 0.0f, (float)P.tiles_x);
    const uint32_t y0 = (uint32_t)raster_clamp(floorf((my - radius) / 16.0f), 0.0f, (float)P.tiles_y);
    const uint32_t y1 = (uint32_t)raster_clamp(floorf((my + radius) / 16.0f) + 1.0f, 0.0f, (float)P.tiles_y);
    if (x0 >= x1 || y0 >= y1) return;
    RasterSplat o;
    o.mx = mx;
    o.my = my;
    const float L = 1.4426950408889634f;
    o.qa = (c / det) * (-0.5f * L);
    o.qb = (-b / det) * -L;
    o.qc = (a / det) * (-0.5f * L);
    o.opacity = s4.w;
    o.rx = x0 | (x1 << 16);
    o.ry = y0 | (y1 << 16);
    o.pad = 0;
    const float* coef = sh + (uint64_t)i * P.stride * 3;
    if (P.color_mode == NPA_RASTER_COLOR_RGB) {
        o.r = coef[0];
        o.g = coef[1];
        o.b = coef[2];
    } else {
        float d[3] = {p.x - P.campos[0], p.y - P.campos[1], p.z - P.campos[2]};
        const float dn = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
#pragma unroll
        for (int k = 0; k < 3; ++k) d[k] = dn > 0.0f ? d[k] / dn : 0.0f;
        // real spherical harmonics, bands 0..3, in the 3DGS sign convention (Condon-Shortley phase)
        const float x = d[0], y = d[1], z = d[2];
        float basis[16];
        basis[0] = 0.28209479177387814f;
        if (P.sh_degree > 0) {
            basis[1] = -0.4886025119029199f * y;
            basis[2] = 0.4886025119029199f * z;
            basis[3] = -0.4886025119029199f * x;
        }
        if (P.sh_degree > 1) {
            const float xx = x * x, yy = y * y, zz = z * z;
            basis[4] = 1.0925484305920792f * (x * y);
            basis[5] = -1.0925484305920792f * (y * z);
            basis[6] = 0.31539156525252005f * (2.0f * zz - xx - yy);
            basis[7] = -1.0925484305920792f * (x * z);
            basis[8] = 0.5462742152960396f * (xx - yy);
            if (P.sh_degree > 2) {
                basis[9] = -0.5900435899266435f * y * (3.0f * xx - yy);
                basis[10] = 2.890611442640554f * (x * y) * z;
                basis[11] = -0.4570457994644658f * y * (4.0f * zz - xx - yy);
                basis[12] = 0.3731763325901154f * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
                basis[13] = -0.4570457994644658f * x * (4.0f * zz - xx - yy);
                basis[14] = 1.445305721320277f * z * (xx - yy);
                basis[15] = -0.5900435899266435f * x * (xx - 3.0f * yy);
            }
        }
        float rgb[3];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < P.K; ++k) acc += basis[k] * coef[k * 3 + ch];
            acc += 0.5f;
            rgb[ch] = acc > 0.0f ? acc : 0.0f;
        }
        o.r = rgb[0];
        o.g = rgb[1];
        o.b = rgb[2];
    }
    out[i] = o;
    ntiles[i] = (x1 - x0) * (y1 - y0);
    dkey[i] = __float_as_uint(tz);
}

__global__ __launch_bounds__(256) void k_raster_gather_counts(const uint32_t* __restrict__ ntiles,
                                                              const uint32_t* __restrict__ order, uint32_t count,
                                                              uint32_t* __restrict__ out) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < count) out[j] = ntiles[order[j]];
}

// The 64-bit sum of the tile counts (the 32-bit scan total can wrap).
__global__ __launch_bounds__(1024) void k_raster_sum64(const uint32_t* __restrict__ in, uint32_t count,
                                                       unsigned long long* __restrict__ total) {
    __shared__ unsigned long long lds[16];
    unsigned long long s = 0;
    for (uint32_t k = threadIdx.x; k < count; k += blockDim.x) s += in[k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (uint32_t w = 0; w < blockDim.x / 64; ++w) t += lds[w];
        *total = t;
    }
}

// kEmitLanes lanes per Gaussian write its (tile, Gaussian) items interleaved, row-major over its
// tile rectangle from start[j].
constexpr uint32_t kEmitLanes = 8;

__global__ __launch_bounds__(256) void k_raster_emit(RasterParams P, const RasterSplat* __restrict__ sp,
                                                     const uint32_t* __restrict__ order,
                                                     const uint32_t* __restrict__ start, uint32_t* __restrict__ keys,
                                                     uint32_t* __restrict__ vals) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t j = t / kEmitLanes;
    const uint32_t sub = (uint32_t)(t % kEmitLanes);
    if (j >= P.count) return;
    const uint32_t begin = start[j], end = start[j + 1];
    if (begin + sub >= end) return;
    const uint32_t g = order[j];
    const uint32_t rx = sp[g].rx, ry = sp[g].ry;
    const uint32_t x0 = rx & 0xffffu, x1 = rx >> 16, y0 = ry & 0xffffu;
    const uint32_t w = x1 - x0;  // >= 1: the Gaussian has items
    uint32_t x = x0 + sub, y = y0;
    while (x >= x1) {
        x -= w;
        ++y;
    }
    for (uint32_t k = begin + sub; k < end; k += kEmitLanes) {
        keys[k] = y * P.tiles_x + x;
        vals[k] = g;
        x += kEmitLanes;
        while (x >= x1) {
            x -= w;
            ++y;
        }
    }
}

__global__ __launch_bounds__(256) void k_raster_tiles(RasterParams P, const RasterSplat* __restrict__ sp,
                                                      const uint32_t* __restrict__ offsets,
                                                      const uint32_t* __restrict__ sorted, float4* __restrict__ image) {
    __shared__ float4 la[256], lb[256];
    __shared__ float lc[256];
    const uint32_t tile = blockIdx.x;
    const uint32_t px = (tile % P.tiles_x) * 16 + (threadIdx.x & 15);
    const uint32_t py = (tile / P.tiles_x) * 16 + (threadIdx.x >> 4);
    const bool inside = px < P.width && py < P.height;
    const float pxc = (float)px + 0.5f, pyc = (float)py + 0.5f;
    const uint32_t begin = offsets[tile], end = offsets[tile + 1];
    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    int done = inside ? 0 : 1;
    for (uint32_t base = begin; base < end; base += 256) {
        if (__syncthreads_count(done) == (int)blockDim.x) break;
        const uint32_t k = base + threadIdx.x;
        if (k < end) {
            const float4* s4 = reinterpret_cast<const float4*>(sp + sorted[k]);
            la[threadIdx.x] = s4[0];
            lb[threadIdx.x] = s4[1];
            lc[threadIdx.x] = s4[2].x;
        }
        __syncthreads();
        const uint32_t n = end - base < 256 ? end - base : 256;
        // Branch-free: every lane evaluates every entry and the tests become selects (the same
        // comparisons, so NaN behaves as in a branching loop); a stopped lane keeps its values.
        // The wave leaves the batch once all of its lanes have stopped.
        for (uint32_t u0 = 0; u0 < n; u0 += 4) {
#pragma unroll
            for (uint32_t du = 0; du < 4; ++du) {
                const uint32_t u = u0 + du;
                if (u >= n) break;  // wave-uniform
                const float4 A = la[u], B = lb[u];  // (mx, my, qa, qb), (qc, opacity, r, g)
                const float C = lc[u];
                const float dx = A.x - pxc, dy = A.y - pyc;
                // power * log2(e), with the oracle's fused operations
                const float p2 = __builtin_fmaf(A.z * dx, dx, __builtin_fmaf(B.x * dy, dy, A.w * dx * dy));
                // the hardware 2^x: below 2^-126 alpha is far under the 1/255 floor either way
                const float alpha = fminf(0.99f, B.y * __builtin_amdgcn_exp2f(p2));
                const float next = T * (1.0f - alpha);
                const bool ok = !done && !(p2 > 0.0f) && !(alpha < 1.0f / 255.0f);
                const bool stop = ok && next < 0.0001f;
                const bool apply = ok && !stop;
                const float wgt = alpha * T;
                cr = apply ? __builtin_fmaf(B.z, wgt, cr) : cr;
                cg = apply ? __builtin_fmaf(B.w, wgt, cg) : cg;
                cb = apply ? __builtin_fmaf(C, wgt, cb) : cb;
                T = apply ? next : T;
                done = done || stop;
            }
            if (__all(done)) break;
        }
    }
    if (inside) image[(uint64_t)py * P.width + px] = make_float4(cr, cg, cb, 1.0f - T);
}

hipError_t launch_raster_gaussians(const float4* pv, const float* sh, const float4* rot, const float4* so,
                                   uint32_t count, const npa_raster_camera& cam, float* image, SplatWorkspace& ws,
                                   hipStream_t stream, Profiler* prof, uint32_t coef_stride) {
    const uint32_t K = (cam.sh_degree + 1) * (cam.sh_degree + 1);
    if (cam.width == 0 || cam.height == 0 || cam.width > kRasterMaxAxis || cam.height > kRasterMaxAxis ||
        cam.sh_degree > 3 || count >= (1u << 31) || (coef_stride != 0 && coef_stride < K))
        return hipErrorInvalidValue;
    RasterParams P{};
    for (int k = 0; k < 12; ++k) P.view[k] = cam.view[k];
    P.fx = cam.fx;
    P.fy = cam.fy;
    P.cx = cam.cx;
    P.cy = cam.cy;
    P.limx = 1.3f * fmaxf(cam.cx, (float)cam.width - cam.cx) / cam.fx;
    P.limy = 1.3f * fmaxf(cam.cy, (float)cam.height - cam.cy) / cam.fy;
    P.near_plane = cam.near_plane;
    P.far_plane = cam.far_plane;
    for (int k = 0; k < 3; ++k)  // camera centre -R^T t
        P.campos[k] = -(cam.view[k] * cam.view[3] + cam.view[4 + k] * cam.view[7] + cam.view[8 + k] * cam.view[11]);
    P.width = cam.width;
    P.height = cam.height;
    P.tiles_x = (cam.width + 15) / 16;
    P.tiles_y = (cam.height + 15) / 16;
    P.count = count;
    P.K = K;
    P.stride = coef_stride ? coef_stride : K;
    P.sh_degree = cam.sh_degree;
    P.color_mode = cam.color_mode;
    const uint32_t ntile_total = P.tiles_x * P.tiles_y;
    if (ntile_total > 65536) return hipErrorInvalidValue;  // the key sort's bin limit
    const uint64_t n1 = count ? count : 1;
    hipError_t e;
#define NPA_RES(buf, n) \
    if ((e = (buf).reserve((size_t)(n))) != hipSuccess) return e;
    NPA_RES(ws.params, n1 * sizeof(RasterSplat));
    NPA_RES(ws.item_start, (4 * n1 + 1) * 4);  // ntiles, depth keys, ordered counts, starts (+1)
    NPA_RES(ws.order, n1 * 4);
    NPA_RES(ws.keys, n1 * 4);
    NPA_RES(ws.offsets, ((uint64_t)ntile_total + 1) * 4);
    NPA_RES(ws.count, 64);
    NPA_RES(ws.scan, (2 * (n1 / kScanBlock + 1) + 2) * 4);
    ProfScope ps(prof, NPA_KERNEL_RASTER, stream);
    RasterSplat* sp = ws.params.as<RasterSplat>();
    uint32_t* ntiles = ws.item_start.as<uint32_t>();
    uint32_t* dkey = ntiles + n1;
    uint32_t* ocounts = dkey + n1;
    uint32_t* start = ocounts + n1;  // n1 + 1 entries
    uint32_t* ord_a = ws.order.as<uint32_t>();
    unsigned long long* d_total64 = reinterpret_cast<unsigned long long*>(ws.count.as<uint32_t>() + 2);
    if (count) {
        hipLaunchKernelGGL(k_raster_prep, dim3((count + 255) / 256), dim3(256), 0, stream, P, pv, sh, rot, so, sp,
                           ntiles, dkey);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    // depth order: stable radix sort of the indices by the depth keys' bits 0-30 (non-negative floats)
    if ((e = sort_index_by_key(dkey, ws.keys.as<uint32_t>(), ord_a, count, 31, ws.sort_temp, stream)) != hipSuccess)
        return e;
    const uint32_t* order = ord_a;
    if (count) {
        hipLaunchKernelGGL(k_raster_gather_counts, dim3((count + 255) / 256), dim3(256), 0, stream, ntiles, order,
                           count, ocounts);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    {  // start = exclusive prefix of the ordered counts; start[count] = total
        const uint32_t nb = (count + kScanBlock - 1) / kScanBlock;
        uint32_t* sums = ws.scan.as<uint32_t>();
        if (nb) {
            hipLaunchKernelGGL(k_scan_partials, dim3(nb), dim3(256), 0, stream, ocounts, count, sums);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k_scan_1block, dim3(1), dim3(1024), 0, stream, sums, sums + nb + 1, nb, start + count);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (nb) {
            hipLaunchKernelGGL(k_scan_apply, dim3(nb), dim3(256), 0, stream, ocounts, start, count, sums + nb + 1);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        hipLaunchKernelGGL(k_raster_sum64, dim3(1), dim3(1024), 0, stream, ocounts, count, d_total64);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    unsigned long long total = 0;
    if ((e = hipMemcpyAsync(&total, d_total64, 8, hipMemcpyDeviceToHost, stream)) != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    if (total >= (1ull << 31)) return hipErrorInvalidValue;  // more (tile, Gaussian) items than the sort takes
    const uint32_t items = (uint32_t)total;
    HashgridPlan plan;
    if (!make_key_sort_plan(items, ntile_total, &plan)) return hipErrorInvalidValue;
    const uint64_t i1 = items ? items : 1;
    NPA_RES(ws.keys, std::max(i1, n1) * 4);
    NPA_RES(ws.vals, i1 * 4);
    NPA_RES(ws.sorted, i1 * 4);
    NPA_RES(ws.ranks, i1 * 4);
    NPA_RES(ws.table, plan.table_entries * 4);
    NPA_RES(ws.totals, (uint64_t)ntile_total * 4);
    NPA_RES(ws.flags, 64);
#undef NPA_RES
    if (count) {
        hipLaunchKernelGGL(k_raster_emit, dim3((uint32_t)(((uint64_t)count * kEmitLanes + 255) / 256)), dim3(256), 0,
                           stream, P, sp, order, start, ws.keys.as<uint32_t>(), ws.vals.as<uint32_t>());
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    // stable counting sort of the items by tile (the scan wrote the item count to start[count])
    e = launch_key_sort(plan, ws.keys.as<uint32_t>(), ws.vals.as<uint32_t>(), start + count, items,
                        ws.ranks.as<uint32_t>(), ws.table.as<uint32_t>(), ws.totals.as<uint32_t>(),
                        ws.offsets.as<uint32_t>(), ws.sorted.as<uint32_t>(), ws.flags.as<uint32_t>(), stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_raster_tiles, dim3(ntile_total), dim3(256), 0, stream, P, sp, ws.offsets.as<uint32_t>(),
                       ws.sorted.as<uint32_t>(), reinterpret_cast<float4*>(image));
    return hipGetLastError();
}

}  // namespace npa
