// npa_perception.hip - SPH neighbour passes and the fused rollout update on gfx950.
//
// Work mapping: the hashgrid build emits one work item per <=64 consecutive sorted
// slots of a bin, so each wavefront's lanes are targets of one bin and (outside hash
// collisions) share the same 3x3(x3) neighbour cells: the neighbour loop runs in
// lockstep and every candidate record / state row is a single broadcast load.
// Each lane accumulates its own sums serially in the reference's neighbour order
// (cells dz, dy, dx; slots ascending = particle index ascending), so the sums are
// bit-identical to the CPU path.
//
//   k_density  rho_i = sum_j W_poly6(r_ij^2)        forward.rs:145-160
//   k_update   second pass (blur, state gradient, density gradient, moment matrix)
//              forward.rs:162-382 -> moment correction, scaling, log-norm
//              normalize.rs:5-118 -> feature row (never stored) -> update MLP
//              model.rs:900-940 -> motion scaling model.rs:867-898 -> 3D gates
//              model.rs:806-837 -> masked Euler step.rs:4-55, written to the
//              ping-pong output in original particle order.
#include <hip/hip_runtime.h>

#include "npa_internal.hpp"

namespace npa {

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

#define NPA_WAVE_LOOP_BEGIN(wl, wl_count)                                       \
    const uint32_t lane = threadIdx.x & 63;                                     \
    const uint32_t wave0 = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); \
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);                      \
    const uint32_t items = *(wl_count);                                         \
    for (uint32_t it = wave0; it < items; it += nwaves) {                       \
        const uint2 item = (wl)[it];                                            \
        if (lane >= item.y) continue;                                           \
        const uint32_t s = item.x + lane;
#define NPA_WAVE_LOOP_END }

template <int D>
__global__ __launch_bounds__(256) void k_density(StepParams P, const float4* __restrict__ srec,
                                                 const int4* __restrict__ scoord,
                                                 const uint32_t* __restrict__ bo,
                                                 const uint32_t* __restrict__ perm,
                                                 const uint2* __restrict__ wl,
                                                 const uint32_t* __restrict__ wl_count,
                                                 float* __restrict__ svol, float* __restrict__ density_out) {
    NPA_WAVE_LOOP_BEGIN(wl, wl_count)
    const uint32_t b = s / P.N;
    float pi[3];
    int ci[3];
    load_rec<D>(srec, scoord, s, pi, ci);
    float rho = 0.0f;
    walk_neighbors<D>(P.g, b, pi, ci, bo, srec, scoord,
                      [&](uint32_t, const float*, float r2) { rho += poly6(r2, P.g); });
    svol[s] = recip_finite(rho);
    if (density_out) density_out[b * P.N + perm[s]] = rho;
    NPA_WAVE_LOOP_END
}

// MODE 0: fused rollout step. MODE 1: perception outputs (features etc.).
template <int D, int SM, int MODE>
__global__ __launch_bounds__(256) void k_update(StepParams P, const float4* __restrict__ srec,
                                                const int4* __restrict__ scoord,
                                                const float* __restrict__ sstate,
                                                const float* __restrict__ svol,
                                                const uint32_t* __restrict__ bo,
                                                const uint32_t* __restrict__ perm,
                                                const uint2* __restrict__ wl,
                                                const uint32_t* __restrict__ wl_count, StepIO io) {
    const uint32_t S = P.S;
    NPA_WAVE_LOOP_BEGIN(wl, wl_count)
    const uint32_t b = s / P.N;
    const uint32_t li = perm[s];
    const uint32_t i = b * P.N + li;
    float pi[3];
    int ci[3];
    load_rec<D>(srec, scoord, s, pi, ci);

    float si[SM], blur[SM], grad[SM * D], dg[D], mom[D * D];
#pragma unroll
    for (int c = 0; c < SM; ++c) {
        si[c] = (uint32_t)c < S ? sstate[(uint64_t)s * S + c] : 0.0f;
        blur[c] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < SM * D; ++k) grad[k] = 0.0f;
#pragma unroll
    for (int k = 0; k < D; ++k) dg[k] = 0.0f;
#pragma unroll
    for (int k = 0; k < D * D; ++k) mom[k] = 0.0f;

    const bool branch_a = P.state_grad && P.density_grad;
    const bool want_sg = P.state_grad != 0, want_dg = P.density_grad != 0;
    const bool want_m = want_sg && P.hybrid;
    walk_neighbors<D>(P.g, b, pi, ci, bo, srec, scoord, [&](uint32_t j, const float* d, float r2) {
        const float vol = svol[j];
        const float smooth = poly6(r2, P.g);
        const float* sj = sstate + (uint64_t)j * S;
        float sv[SM];
#pragma unroll
        for (int c = 0; c < SM; ++c) sv[c] = (uint32_t)c < S ? sj[c] : 0.0f;
        if (branch_a) {  // second_pass_particle forward.rs:263-270
#pragma unroll
            for (int c = 0; c < SM; ++c)
                if ((uint32_t)c < S) blur[c] += sv[c] * smooth * vol;
        } else {  // blur_state forward.rs:174-180
            const float w = smooth * vol;
#pragma unroll
            for (int c = 0; c < SM; ++c)
                if ((uint32_t)c < S) blur[c] += sv[c] * w;
        }
        if (j == s) return;
        if (r2 <= 0.0f) return;  // spiky_gradient_kernel returns zeros (kernels.rs:87-89)
        const float r = sqrtf(r2);
        const float t = P.g.eps - r;
        if (want_dg) {  // spiky_gradient_kernel(coeff = 1)
            const float mag = 1.0f * P.g.k5 * 3.0f * (t * t) / r;
#pragma unroll
            for (int a = 0; a < D; ++a) dg[a] += mag * d[a];
        }
        if (want_sg) {  // spiky_gradient_kernel(coeff = volume_j)
            const float mag = vol * P.g.k5 * 3.0f * (t * t) / r;
            float vg[D];
#pragma unroll
            for (int a = 0; a < D; ++a) vg[a] = mag * d[a];
#pragma unroll
            for (int c = 0; c < SM; ++c) {
                if ((uint32_t)c < S) {
                    const float diff = sv[c] - si[c];
#pragma unroll
                    for (int a = 0; a < D; ++a) grad[c * D + a] += diff * vg[a];
                }
            }
            if (want_m) {
#pragma unroll
                for (int rr = 0; rr < D; ++rr)
#pragma unroll
                    for (int cc = 0; cc < D; ++cc) mom[rr * D + cc] += d[rr] * vg[cc];
            }
        }
    });

    if (want_sg) {
        if (want_m) {  // apply_moment_correction normalize.rs:93-118
            float inv[D * D];
            safe_inverse<D>(mom, inv);
#pragma unroll
            for (int c = 0; c < SM; ++c) {
                float corrected[D];
#pragma unroll
                for (int o = 0; o < D; ++o) corrected[o] = 0.0f;
#pragma unroll
                for (int o = 0; o < D; ++o)
#pragma unroll
                    for (int k = 0; k < D; ++k) corrected[o] += grad[c * D + k] * inv[k * D + o];
#pragma unroll
                for (int o = 0; o < D; ++o) grad[c * D + o] = corrected[o];
            }
        }
#pragma unroll
        for (int c = 0; c < SM; ++c) {  // normalize_state_gradient normalize.rs:5-30
#pragma unroll
            for (int a = 0; a < D; ++a) grad[c * D + a] *= P.state_scale;
            if (P.log_norm_grad) log_normalize<D>(&grad[c * D]);
        }
    }
    if (want_dg) {  // normalize_density_gradient normalize.rs:32-58
#pragma unroll
        for (int a = 0; a < D; ++a) dg[a] *= P.dgrad_scale;
        if (P.log_norm_dgrad) log_normalize<D>(dg);
    }
    const float4 pos4 = io.pos[i];
    const float porig[4] = {pos4.x, pos4.y, pos4.z, pos4.w};

    if constexpr (MODE == 1) {
        // feature assembly forward.rs:100-133
        float* f = io.features + (uint64_t)i * P.F;
        uint32_t off = 0;
#pragma unroll
        for (int c = 0; c < SM; ++c)
            if ((uint32_t)c < S) f[off + c] = si[c];
        off += S;
#pragma unroll
        for (int c = 0; c < SM; ++c)
            if ((uint32_t)c < S) {
                f[off + c] = blur[c];
                if (io.blurred) io.blurred[(uint64_t)i * S + c] = blur[c];
            }
        off += S;
        if (want_sg) {
#pragma unroll
            for (int k = 0; k < SM * D; ++k)
                if ((uint32_t)k < S * D) {
                    f[off + k] = grad[k];
                    if (io.state_gradient) io.state_gradient[(uint64_t)i * S * D + k] = grad[k];
                }
            off += S * D;
        }
        if (want_dg) {
#pragma unroll
            for (int a = 0; a < D; ++a) {
                f[off + a] = dg[a];
                if (io.density_gradient) io.density_gradient[(uint64_t)i * D + a] = dg[a];
            }
            off += D;
        }
        if (P.position_features) {
#pragma unroll
            for (int a = 0; a < D; ++a) f[off + a] = porig[a];
        }
    } else {
        // update MLP forward_update_from_features model.rs:900-940. Each output sum still
        // starts from its bias and adds hidden units in ascending order; the hidden
        // layer is consumed as it is produced instead of being stored.
        constexpr int OM = D + SM;
        const uint32_t O = D + S, F = P.F, H = P.H;
        float u[OM];
#pragma unroll
        for (int o = 0; o < OM; ++o) u[o] = (uint32_t)o < O ? io.b2[o] : 0.0f;
        for (uint32_t h = 0; h < H; ++h) {
            const float* wr = io.w1 + (uint64_t)h * F;
            float sum = io.b1[h];
#pragma unroll
            for (int c = 0; c < SM; ++c)
                if ((uint32_t)c < S) sum += wr[c] * si[c];
#pragma unroll
            for (int c = 0; c < SM; ++c)
                if ((uint32_t)c < S) sum += wr[S + c] * blur[c];
            uint32_t off = 2 * S;
            if (want_sg) {
#pragma unroll
                for (int k = 0; k < SM * D; ++k)
                    if ((uint32_t)k < S * D) sum += wr[off + k] * grad[k];
                off += S * D;
            }
            if (want_dg) {
#pragma unroll
                for (int a = 0; a < D; ++a) sum += wr[off + a] * dg[a];
                off += D;
            }
            if (P.position_features) {
#pragma unroll
                for (int a = 0; a < D; ++a) sum += wr[off + a] * porig[a];
            }
            const float hv = fmaxf(sum, 0.0f);
#pragma unroll
            for (int o = 0; o < OM; ++o)
                if ((uint32_t)o < O) u[o] += io.w2[(uint64_t)o * H + h] * hv;
        }
        // forward_from_features_with_eps model.rs:875-895
        float norm = 0.0f;
#pragma unroll
        for (int a = 0; a < D; ++a) norm += u[a] * u[a];
        norm = sqrtf(norm);
        float dx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int a = 0; a < D; ++a) dx[a] = P.alpha * u[a] * P.motion_eps / (1.0f + norm);
        float sg = 1.0f;
        if (P.gates3d) {  // position-conditioned 3D gates model.rs:806-837, rollout/mod.rs:67-91
            const float liveness = si[3 < SM ? 3 : 0];
            const float sd = si[7 < SM ? 7 : 0];
            sg = clampf_((4.0f - liveness) * 2.0f, 0.0f, 1.0f);
            float mg;
            if (porig[3] >= 0.5f) {
                mg = 0.0f;
            } else {
                const float dgate = clampf_((fabsf(sd) - 0.01f) / 0.02f, 0.0f, 1.0f);
                mg = sg * dgate;
            }
#pragma unroll
            for (int a = 0; a < D; ++a) dx[a] *= mg;
        }
        const float m = io.mask ? io.mask[i]
                                : hash_mask(li, b, P.N, P.update_prob, P.step_index, P.base_seed);
        // euler_step step.rs:31-53
        float pn[4] = {porig[0], porig[1], porig[2], porig[3]};
        constexpr int MEM = D == 3 ? 4 : 2;
#pragma unroll
        for (int a = 0; a < MEM; ++a) pn[a] += P.dt * dx[a] * m;
        if (P.g.boundary == 0) {  // wrap_position hashgrid.rs:183-193
#pragma unroll
            for (int a = 0; a < D; ++a) {
                const float v = pn[a] + P.g.half[a];
                float r = fmodf(v, P.g.extent[a]);
                if (r < 0.0f) r = r + fabsf(P.g.extent[a]);
                pn[a] = r - P.g.half[a];
            }
        }
        io.out_pos[i] = make_float4(pn[0], pn[1], pn[2], pn[3]);
        float* os = io.out_states + (uint64_t)i * S;
#pragma unroll
        for (int c = 0; c < SM; ++c) {
            if ((uint32_t)c < S) {
                float dsc = u[D + c];
                if (P.gates3d) dsc *= sg;
                float next = si[c] + P.dt * dsc * m;
                if (D == 3 && S > 3 && (c == 3 || (S > 8 && c == 8))) next = clampf_(next, -8.0f, 24.0f);
                os[c] = next;
            }
        }
    }
    NPA_WAVE_LOOP_END
}

// forward_from_features_with_eps (model.rs:867-940) for explicit feature rows.
__global__ __launch_bounds__(256) void k_mlp_forward(StepParams P, const float* __restrict__ features,
                                                     uint32_t rows, const float* __restrict__ w1,
                                                     const float* __restrict__ b1,
                                                     const float* __restrict__ w2,
                                                     const float* __restrict__ b2, float* __restrict__ dx,
                                                     float* __restrict__ ds, int dim) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint32_t F = P.F, H = P.H, S = P.S, O = dim + S;
    const float* f = features + (uint64_t)r * F;
    float u[3 + 32];
    for (uint32_t o = 0; o < O; ++o) u[o] = b2[o];
    for (uint32_t h = 0; h < H; ++h) {
        float sum = b1[h];
        const float* wr = w1 + (uint64_t)h * F;
        for (uint32_t k = 0; k < F; ++k) sum += wr[k] * f[k];
        const float hv = fmaxf(sum, 0.0f);
        for (uint32_t o = 0; o < O; ++o) u[o] += w2[(uint64_t)o * H + h] * hv;
    }
    float norm = 0.0f;
    for (int a = 0; a < dim; ++a) norm += u[a] * u[a];
    norm = sqrtf(norm);
    float* px = dx + 4 * (uint64_t)r;
    px[0] = px[1] = px[2] = px[3] = 0.0f;
    for (int a = 0; a < dim; ++a) px[a] = P.alpha * u[a] * P.motion_eps / (1.0f + norm);
    for (uint32_t c = 0; c < S; ++c) ds[(uint64_t)r * S + c] = u[dim + c];
}

// euler_step  crates/burn_automata_kernels/src/reference/step.rs:4-55
__global__ __launch_bounds__(256) void k_euler(GridParams g, const float4* __restrict__ pos,
                                               const float* __restrict__ states,
                                               const float4* __restrict__ dx,
                                               const float* __restrict__ ds,
                                               const float* __restrict__ mask, float dt, uint32_t S,
                                               uint64_t total, float4* __restrict__ out_pos,
                                               float* __restrict__ out_states) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const float m = mask ? mask[i] : 1.0f;
    const float4 p4 = pos[i];
    const float4 d4 = dx[i];
    float p[4] = {p4.x, p4.y, p4.z, p4.w};
    const float d[4] = {d4.x, d4.y, d4.z, d4.w};
    const int mem = g.dim == 3 ? 4 : 2;
    for (int a = 0; a < mem; ++a) p[a] += dt * d[a] * m;
    if (g.boundary == 0) {
        for (int a = 0; a < g.dim; ++a) {
            const float v = p[a] + g.half[a];
            float r = fmodf(v, g.extent[a]);
            if (r < 0.0f) r = r + fabsf(g.extent[a]);
            p[a] = r - g.half[a];
        }
    }
    out_pos[i] = make_float4(p[0], p[1], p[2], p[3]);
    for (uint32_t c = 0; c < S; ++c) {
        float next = states[i * S + c] + dt * ds[i * S + c] * m;
        if (g.dim == 3 && S > 3 && (c == 3 || (S > 8 && c == 8))) next = clampf_(next, -8.0f, 24.0f);
        out_states[i * S + c] = next;
    }
}

__global__ __launch_bounds__(256) void k_update_mask(uint32_t batch, uint32_t n, float p, uint32_t step,
                                                     uint32_t base_seed, float* __restrict__ mask) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)batch * n) return;
    const uint32_t b = (uint32_t)(i / n);
    const uint32_t li = (uint32_t)(i - (uint64_t)b * n);
    mask[i] = hash_mask(li, b, n, p, step, base_seed);
}

// Candidates visited / pairs accepted by the neighbour walk (diagnostic, not on the step path).
template <int D>
__global__ __launch_bounds__(256) void k_count_pairs(StepParams P, const float4* __restrict__ srec,
                                                     const int4* __restrict__ scoord,
                                                     const uint32_t* __restrict__ bo,
                                                     const uint2* __restrict__ wl,
                                                     const uint32_t* __restrict__ wl_count,
                                                     unsigned long long* __restrict__ counters) {
    unsigned long long cand = 0, pairs = 0;
    {
        NPA_WAVE_LOOP_BEGIN(wl, wl_count)
        const uint32_t b = s / P.N;
        float pi[3];
        int ci[3];
        load_rec<D>(srec, scoord, s, pi, ci);
        constexpr int ZLO = D == 3 ? -1 : 0, ZHI = D == 3 ? 1 : 0;
        for (int dz = ZLO; dz <= ZHI; ++dz)
            for (int dy = -1; dy <= 1; ++dy)
                for (int dx = -1; dx <= 1; ++dx) {
                    uint32_t cell;
                    if (!cell_index((int64_t)ci[0] + dx, (int64_t)ci[1] + dy, (int64_t)ci[2] + dz, P.g, &cell))
                        continue;
                    const uint64_t bin = (uint64_t)b * P.g.cells + cell;
                    cand += bo[bin + 1] - bo[bin];
                }
        walk_neighbors<D>(P.g, b, pi, ci, bo, srec, scoord, [&](uint32_t, const float*, float) { pairs += 1; });
        NPA_WAVE_LOOP_END
    }
    atomicAdd(&counters[0], cand);
    atomicAdd(&counters[1], pairs);
}

// Neighbour lists in reference order; write=0 stores per-particle counts, write=1 fills
// indices at the given per-particle offsets (both in original particle order).
template <int D>
__global__ __launch_bounds__(256) void k_neighbor_lists(StepParams P, const float4* __restrict__ srec,
                                                        const int4* __restrict__ scoord,
                                                        const uint32_t* __restrict__ bo,
                                                        const uint32_t* __restrict__ perm,
                                                        const uint2* __restrict__ wl,
                                                        const uint32_t* __restrict__ wl_count,
                                                        uint32_t* __restrict__ counts_or_offsets,
                                                        uint32_t* __restrict__ indices, int write) {
    NPA_WAVE_LOOP_BEGIN(wl, wl_count)
    const uint32_t b = s / P.N;
    const uint32_t i = b * P.N + perm[s];
    float pi[3];
    int ci[3];
    load_rec<D>(srec, scoord, s, pi, ci);
    uint32_t k = write ? counts_or_offsets[i] : 0;
    walk_neighbors<D>(P.g, b, pi, ci, bo, srec, scoord, [&](uint32_t j, const float*, float) {
        if (write) indices[k] = b * P.N + perm[j];
        ++k;
    });
    if (!write) counts_or_offsets[i] = k;
    NPA_WAVE_LOOP_END
}

// ------------------------------------------------------------------ launch
hipError_t launch_density(const StepParams& p, Workspace& ws, float* density_out, int grid_blocks,
                          hipStream_t stream, Profiler* prof) {
    ProfScope ps(prof, NPA_KERNEL_DENSITY, stream);
    if (p.g.dim == 2)
        hipLaunchKernelGGL(k_density<2>, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                           ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), ws.svol.as<float>(),
                           density_out);
    else
        hipLaunchKernelGGL(k_density<3>, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                           ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), ws.svol.as<float>(),
                           density_out);
    return hipGetLastError();
}

template <int D, int SM, int MODE>
static void launch_update_t(const StepParams& p, Workspace& ws, const StepIO& io, int grid_blocks,
                            hipStream_t stream) {
    hipLaunchKernelGGL((k_update<D, SM, MODE>), dim3(grid_blocks), dim3(256), 0, stream, p,
                       ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(),
                       ws.svol.as<float>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                       ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), io);
}

template <int D, int MODE>
static void launch_update_d(const StepParams& p, Workspace& ws, const StepIO& io, int grid_blocks,
                            hipStream_t stream) {
    if (p.S <= 4) launch_update_t<D, 4, MODE>(p, ws, io, grid_blocks, stream);
    else if (p.S <= 8) launch_update_t<D, 8, MODE>(p, ws, io, grid_blocks, stream);
    else if (p.S <= 16) launch_update_t<D, 16, MODE>(p, ws, io, grid_blocks, stream);
    else if (p.S <= 24) launch_update_t<D, 24, MODE>(p, ws, io, grid_blocks, stream);
    else launch_update_t<D, 32, MODE>(p, ws, io, grid_blocks, stream);
}

hipError_t launch_update(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int grid_blocks,
                         hipStream_t stream, Profiler* prof) {
    ProfScope ps(prof, NPA_KERNEL_UPDATE, stream);
    if (p.g.dim == 2) {
        if (mode == 0) launch_update_d<2, 0>(p, ws, io, grid_blocks, stream);
        else launch_update_d<2, 1>(p, ws, io, grid_blocks, stream);
    } else {
        if (mode == 0) launch_update_d<3, 0>(p, ws, io, grid_blocks, stream);
        else launch_update_d<3, 1>(p, ws, io, grid_blocks, stream);
    }
    return hipGetLastError();
}

hipError_t launch_mlp_forward(const StepParams& p, const float* features, uint32_t rows, const StepIO& io,
                              float* dx, float* ds, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(k_mlp_forward, dim3((rows + 255) / 256), dim3(256), 0, stream, p, features, rows,
                       io.w1, io.b1, io.w2, io.b2, dx, ds, p.g.dim);
    return hipGetLastError();
}

hipError_t launch_euler(const StepParams& p, const float4* pos, const float* states, const float4* dx,
                        const float* ds, const float* mask, float4* out_pos, float* out_states,
                        uint64_t total, hipStream_t stream) {
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_euler, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream, p.g, pos, states,
                       dx, ds, mask, p.dt, p.S, total, out_pos, out_states);
    return hipGetLastError();
}

hipError_t launch_update_mask(uint32_t batch, uint32_t n, float prob, uint32_t step, uint32_t base_seed,
                              float* mask, hipStream_t stream) {
    const uint64_t total = (uint64_t)batch * n;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_update_mask, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream, batch, n,
                       prob, step, base_seed, mask);
    return hipGetLastError();
}

hipError_t launch_count_pairs(const StepParams& p, Workspace& ws, int grid_blocks, unsigned long long* counters,
                              hipStream_t stream) {
    if (p.g.dim == 2)
        hipLaunchKernelGGL(k_count_pairs<2>, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.worklist.as<uint2>(),
                           ws.wl_count.as<uint32_t>(), counters);
    else
        hipLaunchKernelGGL(k_count_pairs<3>, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.worklist.as<uint2>(),
                           ws.wl_count.as<uint32_t>(), counters);
    return hipGetLastError();
}

hipError_t launch_neighbor_lists(const StepParams& p, Workspace& ws, uint32_t* counts_or_offsets,
                                 uint32_t* indices, int write, int grid_blocks, hipStream_t stream) {
    if (p.g.dim == 2)
        hipLaunchKernelGGL(k_neighbor_lists<2>, dim3(grid_blocks), dim3(256), 0, stream, p,
                           ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(),
                           ws.perm.as<uint32_t>(), ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(),
                           counts_or_offsets, indices, write);
    else
        hipLaunchKernelGGL(k_neighbor_lists<3>, dim3(grid_blocks), dim3(256), 0, stream, p,
                           ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(),
                           ws.perm.as<uint32_t>(), ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(),
                           counts_or_offsets, indices, write);
    return hipGetLastError();
}

}  // namespace npa
