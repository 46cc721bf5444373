// npa_device.hpp - device-side building blocks shared by the NPA kernels (gfx950, wave64).
//
// Numerics: every expression keeps the association order of the reference Rust
// source it follows (cited per function) and the library is compiled with
// -ffp-contract=off, so no a*b+c is fused. f32 division and sqrt are the
// IEEE-correct sequences hipcc emits by default.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "npa_math.hpp"

namespace npa {

constexpr int kWave = 64;

// Uniform parameters of a hashgrid (HashGridConfig plus derived constants).
struct GridParams {
    int dim;         // 2 or 3
    int boundary;    // 0 periodic, 1 clamped
    int mode;        // 0 grid, 1 particle
    uint32_t size[3];
    uint32_t cells;  // cells per system
    float eps;
    float eps2;      // eps * eps
    float extent[3]; // size[a] as f32 * eps
    float half[3];   // extent * 0.5
    float k6;        // poly6 normalisation
    float k5;        // spiky-gradient normalisation
    // Particle mode: 0 - bins by the reference's mixing hash (particle_cell_hash, hashgrid.rs:147-153),
    // as npa_build_hashgrid exposes them; 1 - bins by the cell coordinates modulo the grid size, for
    // the step's own sort. Every neighbour visit looks a cell up by its coordinates and keeps only
    // that cell's particles, so which cells share a bin changes no result; with coordinate bins a
    // cloud narrower than the grid puts one cell in each bin, and consecutive bins are neighbouring
    // cells.
    int spatial;
};

// Wave-level scans and reductions through DPP: row_shr within each 16-lane row, then row_bcast:15
// and row_bcast:31 across the rows (a generic shuffle compiles to ds_bpermute, an LDS round trip per
// step). A lane whose DPP source is outside its row, or whose row the row mask leaves out, adds the
// identity.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_or_identity(uint32_t identity, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROWS, 0xf, false);
}
// inclusive prefix sum over each 16-lane row
__device__ __forceinline__ uint32_t row_incl_add(uint32_t v) {
    v += dpp_or_identity<0x111, 0xf>(0u, v);
    v += dpp_or_identity<0x112, 0xf>(0u, v);
    v += dpp_or_identity<0x114, 0xf>(0u, v);
    v += dpp_or_identity<0x118, 0xf>(0u, v);
    return v;
}
// inclusive prefix sum over the wave's 64 lanes
__device__ __forceinline__ uint32_t wave_incl_add(uint32_t v) {
    v = row_incl_add(v);
    v += dpp_or_identity<0x142, 0xa>(0u, v);  // rows 1, 3 add lane 15, 47
    v += dpp_or_identity<0x143, 0xc>(0u, v);  // rows 2, 3 add lane 31
    return v;
}
// the wave's minimum / maximum (wave-uniform): quads, half rows, rows, then across the rows into
// lane 63
__device__ __forceinline__ int wave_min_i32(int v) {
    constexpr uint32_t id = 0x7fffffffu;
    v = min(v, (int)dpp_or_identity<0xb1, 0xf>(id, (uint32_t)v));   // quad_perm [1,0,3,2]
    v = min(v, (int)dpp_or_identity<0x4e, 0xf>(id, (uint32_t)v));   // quad_perm [2,3,0,1]
    v = min(v, (int)dpp_or_identity<0x141, 0xf>(id, (uint32_t)v));  // row_half_mirror
    v = min(v, (int)dpp_or_identity<0x140, 0xf>(id, (uint32_t)v));  // row_mirror
    v = min(v, (int)dpp_or_identity<0x142, 0xa>(id, (uint32_t)v));  // row_bcast:15
    v = min(v, (int)dpp_or_identity<0x143, 0xc>(id, (uint32_t)v));  // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max_i32(int v) {
    constexpr uint32_t id = 0x80000000u;
    v = max(v, (int)dpp_or_identity<0xb1, 0xf>(id, (uint32_t)v));
    v = max(v, (int)dpp_or_identity<0x4e, 0xf>(id, (uint32_t)v));
    v = max(v, (int)dpp_or_identity<0x141, 0xf>(id, (uint32_t)v));
    v = max(v, (int)dpp_or_identity<0x140, 0xf>(id, (uint32_t)v));
    v = max(v, (int)dpp_or_identity<0x142, 0xa>(id, (uint32_t)v));
    v = max(v, (int)dpp_or_identity<0x143, 0xc>(id, (uint32_t)v));
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_or_identity<0xb1, 0xf>(0u, v));
    v = max(v, dpp_or_identity<0x4e, 0xf>(0u, v));
    v = max(v, dpp_or_identity<0x141, 0xf>(0u, v));
    v = max(v, dpp_or_identity<0x140, 0xf>(0u, v));
    v = max(v, dpp_or_identity<0x142, 0xa>(0u, v));
    v = max(v, dpp_or_identity<0x143, 0xc>(0u, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// the wave's sum (wave-uniform)
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
    v += dpp_or_identity<0xb1, 0xf>(0u, v);
    v += dpp_or_identity<0x4e, 0xf>(0u, v);
    v += dpp_or_identity<0x141, 0xf>(0u, v);
    v += dpp_or_identity<0x140, 0xf>(0u, v);
    v += dpp_or_identity<0x142, 0xa>(0u, v);
    v += dpp_or_identity<0x143, 0xc>(0u, v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Rust `f as isize` of a floored f32: saturating, NaN -> 0.
__device__ __forceinline__ int64_t f32_to_isize(float f) {
    if (f != f) return 0;
    if (f >= 9223372036854775808.0f) return INT64_MAX;
    if (f <= -9223372036854775808.0f) return INT64_MIN;
    return (int64_t)f;
}

__device__ __forceinline__ int64_t rem_euclid_i64(int64_t a, int64_t m) {
    int64_t r = a % m;
    return r < 0 ? r + m : r;
}

// mix_coord  crates/burn_automata_kernels/src/hashgrid.rs:155-163
__device__ __forceinline__ uint32_t mix_coord(int64_t value, uint32_t salt) {
    uint32_t x = ((uint32_t)(int32_t)value) ^ salt;
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// particle_cell_hash  hashgrid.rs:147-153
__device__ __forceinline__ uint32_t particle_hash(int64_t c0, int64_t c1, int64_t c2, const GridParams& g) {
    if (g.spatial) {  // coordinate bins (see GridParams::spatial)
        auto wrap = [](int64_t c, uint32_t m) -> uint32_t {  // Euclidean remainder; a mask for 2^k
            return (m & (m - 1)) == 0 ? (uint32_t)c & (m - 1) : (uint32_t)rem_euclid_i64(c, m);
        };
        uint32_t h = wrap(c0, g.size[0]) + g.size[0] * wrap(c1, g.size[1]);
        if (g.dim == 3) h += g.size[0] * g.size[1] * wrap(c2, g.size[2]);
        return h;
    }
    uint32_t h = mix_coord(c0, 0x9e3779b9u) ^ mix_coord(c1, 0x85ebca6bu);
    if (g.dim == 3) h ^= mix_coord(c2, 0xc2b2ae35u);
    return h % g.cells;
}

// Largest |coordinate| the device path stores exactly in an i32 and can offset by +-1.
constexpr int64_t kCoordLimit = (int64_t)1 << 30;

// cell_coords_for_position  hashgrid.rs:98-121. Sets *overflow when a Particle-mode
// coordinate leaves +-2^30 (the i32 records would no longer be exact).
__device__ __forceinline__ void cell_coords(const float* p, const GridParams& g, int64_t c[3], bool* overflow) {
    c[0] = c[1] = c[2] = 0;
    for (int a = 0; a < g.dim; ++a) {
        if (g.mode == 1) {
            int64_t v = f32_to_isize(floorf(p[a] / g.eps));
            if (v > kCoordLimit || v < -kCoordLimit) *overflow = true;
            c[a] = v;
            continue;
        }
        int64_t size = (int64_t)g.size[a];
        int64_t cell = f32_to_isize(floorf((p[a] + g.half[a]) / g.eps));
        if (g.boundary == 0) {
            cell = rem_euclid_i64(cell, size);
        } else {
            if (cell < 0) cell = 0;
            if (cell > size - 1) cell = size - 1;
        }
        c[a] = cell;
    }
}

// cell_index_from_coords  hashgrid.rs:123-145 (false = None).
__device__ __forceinline__ bool cell_index(int64_t c0, int64_t c1, int64_t c2, const GridParams& g, uint32_t* out) {
    if (g.mode == 1) {
        *out = particle_hash(c0, c1, c2, g);
        return true;
    }
    int64_t cs[3] = {c0, c1, c2};
    uint32_t stride = 1, hash = 0;
    for (int a = 0; a < g.dim; ++a) {
        int64_t size = (int64_t)g.size[a];
        int64_t cell;
        if (g.boundary == 0) {
            cell = rem_euclid_i64(cs[a], size);
        } else {
            if (cs[a] < 0 || cs[a] >= size) return false;
            cell = cs[a];
        }
        hash += (uint32_t)cell * stride;
        stride *= (uint32_t)size;
    }
    *out = hash;
    return true;
}

// cell_for_position  hashgrid.rs:71-96 (coords as computed above).
__device__ __forceinline__ uint32_t cell_of_coords(const int64_t c[3], const GridParams& g) {
    uint32_t out = 0;
    cell_index(c[0], c[1], c[2], g, &out);  // in-range by construction for Grid mode
    return out;
}

// neighbor_delta  hashgrid.rs:165-181, component a.
// Branch-free: both wrapped candidates are computed and one is selected (same values as the
// reference's if / else-if, NaN included).
__device__ __forceinline__ float delta_axis(float pi, float pj, int a, const GridParams& g) {
    const float v = pj - pi;
    if (g.boundary == 0) {  // wave-uniform
        const float up = v - g.extent[a], dn = v + g.extent[a];
        return v > g.half[a] ? up : (v < -g.half[a] ? dn : v);
    }
    return v;
}

// smoothing_poly6_kernel  crates/burn_automata_kernels/src/reference/kernels.rs:51-58
__device__ __forceinline__ float poly6(float r2, const GridParams& g) {
    const float x = g.eps2 - r2;
    const float w = g.k6 * x * x * x;
    return r2 >= g.eps2 ? 0.0f : w;
}

// RecipFinite::recip_finite  kernels.rs:146-154
__device__ __forceinline__ float recip_finite(float x) {
    if (fabsf(x) <= 1e-20f || !isfinite(x)) return 0.0f;
    return 1.0f / x;
}

// log_normalize_vector  crates/burn_automata_kernels/src/reference/normalize.rs:60-69
template <int N>
__device__ __forceinline__ void log_normalize(float* v) {
    const float E = 1.0e-6f;
    float s = v[0] * v[0];
#pragma unroll
    for (int k = 1; k < N; ++k) s += v[k] * v[k];
    float norm = fmaxf(sqrtf(s + E * E), E);
    float scale = npa_log1pf(norm) / norm;  // host-libm-identical log1pf (npa_math.hpp)
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] *= scale;
}

// safe_inverse_symmetric  kernels.rs:3-49 (row-major D x D in, out)
template <int D>
__device__ __forceinline__ void safe_inverse(const float* m, float* out) {
    const float TOL = 1e-3f;
#pragma unroll
    for (int k = 0; k < D * D; ++k) out[k] = 0.0f;
    if constexpr (D == 2) {
        float a = m[0], b = m[1], d = m[3];
        float det = a * d - b * b;
        if (fabsf(det) < TOL) {
            out[0] = 1.0f;
            out[3] = 1.0f;
            return;
        }
        float inv = 1.0f / det;
        out[0] = d * inv;
        out[1] = -b * inv;
        out[2] = -b * inv;
        out[3] = a * inv;
    } else {
        float a = m[0], b = m[1], c = m[2], d = m[4], e = m[5], f = m[8];
        float t1 = d * f - e * e;
        float t2 = c * e - b * f;
        float t3 = b * e - c * d;
        float det = a * t1 + b * t2 + c * t3;
        if (fabsf(det) < TOL) {
            out[0] = 1.0f;
            out[4] = 1.0f;
            out[8] = 1.0f;
            return;
        }
        float inv = 1.0f / det;
        out[0] = t1 * inv;
        out[1] = t2 * inv;
        out[2] = t3 * inv;
        out[3] = t2 * inv;
        out[4] = (a * f - c * c) * inv;
        out[5] = (b * c - a * e) * inv;
        out[6] = t3 * inv;
        out[7] = (b * c - a * e) * inv;
        out[8] = (a * d - b * b) * inv;
    }
}

// hash_u32 / random01  crates/burn_automata/src/gpu_step.wgsl:1019-1031
__device__ __forceinline__ uint32_t hash_u32(uint32_t x) {
    x = (x ^ 61u) ^ (x >> 16);
    x = x + (x << 3);
    x = x ^ (x >> 4);
    x = x * 0x27d4eb2du;
    x = x ^ (x >> 15);
    return x;
}

__device__ __forceinline__ float random01(uint32_t particle, uint32_t step, uint32_t seed) {
    uint32_t mixed = hash_u32(particle ^ hash_u32(step + 0x9e3779b9u) ^ seed);
    return (float)(mixed >> 8) * (1.0f / 16777216.0f);
}

// update_mask  gpu_step.wgsl:1033-1056 with lane seed base ^ (lane * N).
__device__ __forceinline__ float hash_mask(uint32_t local, uint32_t lane, uint32_t particle_count,
                                           float p, uint32_t step, uint32_t base_seed) {
    if (p >= 1.0f) return 1.0f;
    if (p <= 0.0f) return 0.0f;
    uint32_t seed = base_seed ^ (lane * particle_count);
    return random01(local, step, seed) < p ? 1.0f : 0.0f;
}

__device__ __forceinline__ float clampf_(float v, float lo, float hi) {  // f32::clamp
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

// wrap_position  crates/burn_automata_kernels/src/hashgrid.rs:183-193, axis a of a periodic grid:
// (v + half).rem_euclid(extent) - half.
__device__ __forceinline__ float wrap_axis(float v, int a, const GridParams& g) {
    const float x = v + g.half[a];
    float r = fmodf(x, g.extent[a]);
    if (r < 0.0f) r = r + fabsf(g.extent[a]);
    return r - g.half[a];
}

// The opacity-logit channels euler_step clamps in 3D (step.rs:47-50, GROWTH_3D_*_OPACITY_LOGIT
// types.rs:1-2).
__device__ __forceinline__ bool clamped_channel(int dim, uint32_t S, uint32_t c) {
    return dim == 3 && S > 3 && (c == 3 || (S > 8 && c == 8));
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    uint32_t lane = __lane_id();
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Sorted-record access and the reference's neighbour walk, shared by the step and adjoint passes.
template <int D>
__device__ __forceinline__ void load_rec(const float4* __restrict__ srec, const int4* __restrict__ scoord,
                                         uint32_t j, float* p, int* c) {
    const float4 r = srec[j];
    if constexpr (D == 2) {
        p[0] = r.x;
        p[1] = r.y;
        p[2] = 0.0f;
        c[0] = __float_as_int(r.z);
        c[1] = __float_as_int(r.w);
        c[2] = 0;
    } else {
        p[0] = r.x;
        p[1] = r.y;
        p[2] = r.z;
        const int4 q = scoord[j];
        c[0] = q.x;
        c[1] = q.y;
        c[2] = q.z;
    }
}

// for_each_neighbor  crates/burn_automata_kernels/src/reference/neighbor.rs:3-44
template <int D, class Body>
__device__ __forceinline__ void walk_neighbors(const GridParams& g, uint32_t b, const float* pi, const int* ci,
                                               const uint32_t* __restrict__ bo,
                                               const float4* __restrict__ srec,
                                               const int4* __restrict__ scoord, Body&& body) {
    constexpr int ZLO = D == 3 ? -1 : 0, ZHI = D == 3 ? 1 : 0;
    for (int dz = ZLO; dz <= ZHI; ++dz)
        for (int dy = -1; dy <= 1; ++dy)
            for (int dx = -1; dx <= 1; ++dx) {
                const int64_t n0 = (int64_t)ci[0] + dx, n1 = (int64_t)ci[1] + dy, n2 = (int64_t)ci[2] + dz;
                uint32_t cell;
                if (!cell_index(n0, n1, n2, g, &cell)) continue;
                const uint64_t bin = (uint64_t)b * g.cells + cell;
                const uint32_t beg = bo[bin], end = bo[bin + 1];
                for (uint32_t j = beg; j < end; ++j) {
                    float pj[3];
                    int cj[3];
                    load_rec<D>(srec, scoord, j, pj, cj);
                    if (g.mode == 1) {
                        if ((int64_t)cj[0] != n0 || (int64_t)cj[1] != n1) continue;
                        if (D == 3 && (int64_t)cj[2] != n2) continue;
                    }
                    float d[3];
                    d[0] = delta_axis(pi[0], pj[0], 0, g);
                    d[1] = delta_axis(pi[1], pj[1], 1, g);
                    float r2 = d[0] * d[0];
                    r2 += d[1] * d[1];
                    if constexpr (D == 3) {
                        d[2] = delta_axis(pi[2], pj[2], 2, g);
                        r2 += d[2] * d[2];
                    } else {
                        d[2] = 0.0f;
                    }
                    if (r2 < g.eps2) body(j, d, r2);
                }
            }
}

}  // namespace npa
