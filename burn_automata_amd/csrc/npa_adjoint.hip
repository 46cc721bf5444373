// npa_adjoint.hip - the perception adjoint (reverse mode of perceive_with_options) on gfx950.
//
// Reference: perceive_adjoint_with_options, crates/burn_automata_kernels/src/reference/adjoint.rs.
// The reference walks every particle idx once and scatters into the adjoint arrays of idx and of
// its neighbours j. Here every particle gathers instead: the neighbour relation is symmetric
// with equal multiplicity (for_each_neighbor accepts j for idx exactly when it accepts idx for j:
// the same cell offsets negated, the same r^2 < eps^2 test on the negated delta), so a particle
// k receives, walking its own neighbour list, every term the reference adds into k - both the
// terms of the pairs where k is the neighbour j of idx = that neighbour, and the terms where k
// is idx. No atomics; the result is deterministic and equals the reference's up to rounding:
// each particle adds its terms in its own neighbour order, and the state-gradient terms of a pair
// sum their channels' gradient adjoints before the (linear) spiky delta adjoint, which the
// reference applies once per channel.
//
//   k_adj_density  rho_k over the walk, as the forward density pass          forward.rs:145-160
//   k_adj_prep     per particle: the forward state-gradient sums and moment matrix, then the
//                  adjoint of moment correction / scaling / log-norm (raw-gradient adjoint,
//                  moment adjoint) and of the density gradient                adjoint.rs:168-397
//   k_adj_gather   per particle: blurred-state, state-gradient, hybrid-moment and
//                  density-gradient pair terms in both roles; identity and position rows;
//                  the particle's density adjoint                             adjoint.rs:27-348
//   k_adj_density_kernel  the density kernel's position terms                 adjoint.rs:399-418
#include <hip/hip_runtime.h>

#include "npa_internal.hpp"

namespace npa {

// spiky_gradient_kernel  kernels.rs:81-98
template <int D>
__device__ __forceinline__ void spiky(const float* d, float r2, const GridParams& g, float coeff, float* out) {
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = 0.0f;
    if (r2 <= 0.0f || r2 >= g.eps2) return;
    const float r = sqrtf(r2);
    const float t = g.eps - r;
    const float mag = coeff * g.k5 * 3.0f * (t * t) / r;
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = mag * d[a];
}

// smoothing_poly6_delta_adjoint  kernels.rs:62-79
template <int D>
__device__ __forceinline__ void poly6_delta_adjoint(const float* d, float r2, const GridParams& g, float adj,
                                                    float* out) {
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = 0.0f;
    if (r2 >= g.eps2) return;
    const float x = g.eps2 - r2;
    const float dk = -3.0f * g.k6 * x * x;
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = adj * dk * 2.0f * d[a];
}

// log_normalize_adjoint  normalize.rs:71-91 (adds into in_adj)
template <int D>
__device__ __forceinline__ void log_normalize_adjoint(const float* in, const float* out_adj, float* in_adj) {
    const float E = 1.0e-6f;
    float s = in[0] * in[0];
#pragma unroll
    for (int k = 1; k < D; ++k) s += in[k] * in[k];
    const float norm = fmaxf(sqrtf(s + E * E), E);
    const float lp = npa_log1pf(norm);
    const float scale = lp / norm;
    const float dscale = (norm / (1.0f + norm) - lp) / (norm * norm);
    float dot = in[0] * out_adj[0];
#pragma unroll
    for (int k = 1; k < D; ++k) dot += in[k] * out_adj[k];
    const float radial = dscale * dot / norm;
#pragma unroll
    for (int k = 0; k < D; ++k) in_adj[k] += scale * out_adj[k] + radial * in[k];
}

// accumulate_volume_density_adjoint  adjoint.rs:420-431
__device__ __forceinline__ void volume_density_adjoint(float rho, float v_adj, float* acc) {
    if (fabsf(rho) <= 1.0e-20f || !isfinite(rho)) return;
    *acc -= v_adj / (rho * rho);
}

struct AdjointArgs {
    const float4* srec;
    const int4* scoord;
    const uint32_t* bo;
    const uint32_t* perm;
    const float* sstate;  // [T][SS] sorted, padded
    const float* fadj;    // [T][F] particle order
    float* sdens;         // [T] slot order
    float* sfb;           // [T][SS] blurred-feature adjoint rows, slot order
    float* rga;           // [T][SS * D] raw state-gradient adjoint, slot order
    float* madj;          // [T][9] moment adjoint
    float* rda;           // [T][4] raw density-gradient adjoint
    float* dadj;          // [T] density adjoint
    float4* ppos;         // [T] position adjoint before the density-kernel terms, slot order
    float* state_adj;     // [T][S] particle order (output)
    float4* pos_adj;      // [T] particle order (output)
};

template <int D>
__global__ __launch_bounds__(256) void k_adj_density(StepParams P, AdjointArgs A) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= P.T) return;
    const uint32_t b = s / P.N;
    float pi[3];
    int ci[3];
    load_rec<D>(A.srec, A.scoord, s, pi, ci);
    float rho = 0.0f;
    walk_neighbors<D>(P.g, b, pi, ci, A.bo, A.srec, A.scoord, [&](uint32_t, const float*, float r2) {
        rho += poly6(r2, P.g);
    });
    A.sdens[s] = rho;
}

// A particle's channels are split over a group of L = SM / kCpl lanes (lane l owns channels
// l * kCpl .. l * kCpl + kCpl - 1): pair-level quantities are computed by every lane of the group,
// per-channel terms by the channel's lane, and sums across channels are combined in a fixed
// butterfly within the group, so results stay deterministic.
constexpr int kCpl = 4;

template <int L>
__device__ __forceinline__ float group_sum(float v) {
    // butterfly: partner lane ^ m for m = L/2, ..., 1 (the same pairing in every lane, so each lane
    // ends with the same sum); m < 4 stays within a quad and travels by DPP quad_perm
#pragma unroll
    for (int m = L / 2; m >= 4; m >>= 1) v += __shfl_xor(v, m, L);
    if constexpr (L >= 4) v += __int_as_float((int)dpp_or_identity<0x4e, 0xf>(0u, (uint32_t)__float_as_int(v)));  // lane ^ 2
    if constexpr (L >= 2) v += __int_as_float((int)dpp_or_identity<0xb1, 0xf>(0u, (uint32_t)__float_as_int(v)));  // lane ^ 1
    return v;
}

// spiky_gradient_delta_adjoint (kernels.rs:100-126), split: its pair-level part for one
// coefficient (spiky_pre) and the per-channel part - the same operations on the same values as
// the reference's one call per channel.
struct SpikyPre {
    float r, scale, dscale;
    bool live;
};
__device__ __forceinline__ SpikyPre spiky_pre(float r2, const GridParams& g, float coeff) {
    SpikyPre q{0.0f, 0.0f, 0.0f, false};
    if (r2 <= 0.0f || r2 >= g.eps2) return q;
    q.live = true;
    q.r = sqrtf(r2);
    const float norm = coeff * g.k5 * 3.0f;
    const float t = g.eps - q.r;
    q.scale = norm * (t * t) / q.r;
    q.dscale = norm * (1.0f - (g.eps * g.eps) / r2);
    return q;
}
template <int D>
__device__ __forceinline__ void spiky_delta_adjoint_pre(const float* d, const SpikyPre& q, const float* adj,
                                                        float* out) {
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = 0.0f;
    if (!q.live) return;
    float dot = adj[0] * d[0];
#pragma unroll
    for (int a = 1; a < D; ++a) dot += adj[a] * d[a];
#pragma unroll
    for (int a = 0; a < D; ++a) out[a] = q.scale * adj[a] + q.dscale * dot * d[a] / q.r;
}

template <int D, int SM>
__global__ __launch_bounds__(256) void k_adj_prep(StepParams P, AdjointArgs A) {
    constexpr int L = SM / kCpl;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t s = t / L, lane = t % L;
    if (s >= P.T) return;  // whole groups leave together
    const uint32_t b = s / P.N;
    const uint64_t pk = (uint64_t)b * P.N + A.perm[s];
    const uint32_t S = P.S;
    const int c0 = (int)lane * kCpl;
    const float* fa = A.fadj + pk * P.F;
#pragma unroll
    for (int u = 0; u < kCpl; ++u)
        if (c0 + u < (int)S) A.sfb[(uint64_t)s * P.SS + c0 + u] = fa[S + c0 + u];
    float pi[3];
    int ci[3];
    load_rec<D>(A.srec, A.scoord, s, pi, ci);
    const bool rowlane = c0 < (int)P.SS;  // lanes past the padded row (S <= 4 or S > 16) own no channel
    const float* si = A.sstate + (uint64_t)s * P.SS + c0;
    uint32_t cur = 2 * S;
    if (P.state_grad) {
        float raw[kCpl * D];
        float moment[D * D];
#pragma unroll
        for (int k = 0; k < kCpl * D; ++k) raw[k] = 0.0f;
#pragma unroll
        for (int k = 0; k < D * D; ++k) moment[k] = 0.0f;
        walk_neighbors<D>(P.g, b, pi, ci, A.bo, A.srec, A.scoord, [&](uint32_t j, const float* d, float r2) {
            if (j == s) return;
            const float vol = recip_finite(A.sdens[j]);
            float g[D];
            spiky<D>(d, r2, P.g, vol, g);
            if (rowlane) {
                const float* sj = A.sstate + (uint64_t)j * P.SS + c0;
#pragma unroll
                for (int u = 0; u < kCpl; ++u) {
                    const float diff = sj[u] - si[u];
#pragma unroll
                    for (int a = 0; a < D; ++a) raw[u * D + a] += diff * g[a];
                }
            }
            if (P.hybrid) {
#pragma unroll
                for (int r = 0; r < D; ++r)
#pragma unroll
                    for (int cc = 0; cc < D; ++cc) moment[r * D + cc] += d[r] * g[cc];
            }
        });
        float inv[D * D];
        if (P.hybrid) safe_inverse<D>(moment, inv);
        const float scale = P.state_scale;
        float inv_adj[D * D];
#pragma unroll
        for (int k = 0; k < D * D; ++k) inv_adj[k] = 0.0f;
        const float* gadj = fa + cur;
        float* rg = A.rga + (uint64_t)s * P.SS * D;
#pragma unroll
        for (int u = 0; u < kCpl; ++u) {
            const int c = c0 + u;
            if (c >= (int)S) continue;
            float corr[D];
#pragma unroll
            for (int a = 0; a < D; ++a) corr[a] = raw[u * D + a];
            if (P.hybrid) {
                float mc[D];
#pragma unroll
                for (int o = 0; o < D; ++o) mc[o] = 0.0f;
#pragma unroll
                for (int o = 0; o < D; ++o)
#pragma unroll
                    for (int ia = 0; ia < D; ++ia) mc[o] += corr[ia] * inv[ia * D + o];
#pragma unroll
                for (int a = 0; a < D; ++a) corr[a] = mc[a];
            }
            float nin[D], cadj[D], ga[D];
#pragma unroll
            for (int a = 0; a < D; ++a) {
                nin[a] = corr[a] * scale;
                ga[a] = gadj[c * D + a];
                cadj[a] = 0.0f;
            }
            if (P.log_norm_grad) log_normalize_adjoint<D>(nin, ga, cadj);
            else
#pragma unroll
                for (int a = 0; a < D; ++a) cadj[a] = ga[a];
#pragma unroll
            for (int a = 0; a < D; ++a) cadj[a] *= scale;
            float radj[D];
            if (P.hybrid) {
#pragma unroll
                for (int ia = 0; ia < D; ++ia) radj[ia] = 0.0f;
#pragma unroll
                for (int ia = 0; ia < D; ++ia)
#pragma unroll
                    for (int o = 0; o < D; ++o) radj[ia] += cadj[o] * inv[ia * D + o];
#pragma unroll
                for (int ia = 0; ia < D; ++ia)
#pragma unroll
                    for (int o = 0; o < D; ++o) inv_adj[ia * D + o] += raw[u * D + ia] * cadj[o];
            } else {
#pragma unroll
                for (int a = 0; a < D; ++a) radj[a] = cadj[a];
            }
#pragma unroll
            for (int a = 0; a < D; ++a) rg[c * D + a] = radj[a];
        }
        if (P.hybrid) {  // inverse_matrix_adjoint  adjoint.rs:447-468, inv_adj summed over the group
#pragma unroll
            for (int k = 0; k < D * D; ++k) inv_adj[k] = group_sum<L>(inv_adj[k]);
            if (lane == 0) {
                float* m = A.madj + (uint64_t)s * 9;
#pragma unroll
                for (int row = 0; row < D; ++row)
#pragma unroll
                    for (int col = 0; col < D; ++col) {
                        float v = 0.0f;
#pragma unroll
                        for (int ir = 0; ir < D; ++ir)
#pragma unroll
                            for (int ic = 0; ic < D; ++ic) v += inv[ir * D + row] * inv_adj[ir * D + ic] * inv[col * D + ic];
                        m[row * D + col] = 0.0f - v;
                    }
            }
        }
        cur += S * D;
    }
    if (P.density_grad && lane == 0) {  // adjoint.rs:350-397
        float rawd[D];
#pragma unroll
        for (int a = 0; a < D; ++a) rawd[a] = 0.0f;
        walk_neighbors<D>(P.g, b, pi, ci, A.bo, A.srec, A.scoord, [&](uint32_t j, const float* d, float r2) {
            if (j == s) return;
            float g[D];
            spiky<D>(d, r2, P.g, 1.0f, g);
#pragma unroll
            for (int a = 0; a < D; ++a) rawd[a] += g[a];
        });
        const float scale = P.dgrad_scale;
        float nin[D], radj[D], da[D];
#pragma unroll
        for (int a = 0; a < D; ++a) {
            nin[a] = rawd[a] * scale;
            radj[a] = 0.0f;
            da[a] = fa[cur + a];
        }
        if (P.log_norm_dgrad) {
            log_normalize_adjoint<D>(nin, da, radj);
#pragma unroll
            for (int a = 0; a < D; ++a) radj[a] *= scale;
        } else {
#pragma unroll
            for (int a = 0; a < D; ++a) radj[a] = da[a] * scale;
        }
#pragma unroll
        for (int a = 0; a < D; ++a) A.rda[(uint64_t)s * 4 + a] = radj[a];
    }
}

// The pair terms of both roles, gathered by the receiving particle k (slot s). For a neighbour j
// with delta d = p_j - p_k, the pair seen from j is delta -d (exact: IEEE subtraction and the
// periodic wrap are sign-symmetric) with the same r^2. Pair-level terms are added by lane 0 of
// the group, per-channel terms by the channel's lane; the position and density adjoints are
// summed over the group at the end.
template <int D, int SM>
__global__ __launch_bounds__(256) void k_adj_gather(StepParams P, AdjointArgs A) {
    constexpr int L = SM / kCpl;
    const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t s = tid / L, lane = tid % L;
    if (s >= P.T) return;  // whole groups leave together
    const uint32_t b = s / P.N;
    const uint64_t pk = (uint64_t)b * P.N + A.perm[s];
    const uint32_t S = P.S;
    const int c0 = (int)lane * kCpl;
    const bool lead = lane == 0;
    const bool rowlane = c0 < (int)P.SS;  // lanes past the padded row own no channel
    const float* fa = A.fadj + pk * P.F;
    float acc[kCpl], sk[kCpl], fbk[kCpl];
#pragma unroll
    for (int u = 0; u < kCpl; ++u) {
        const int c = c0 + u;
        acc[u] = c < (int)S ? fa[c] : 0.0f;  // the identity rows (adjoint.rs:68-71)
        sk[u] = rowlane ? A.sstate[(uint64_t)s * P.SS + c] : 0.0f;
        fbk[u] = c < (int)S ? A.sfb[(uint64_t)s * P.SS + c] : 0.0f;
    }
    const float rho_k = A.sdens[s];
    const float vol_k = recip_finite(rho_k);
    float pa[D];
#pragma unroll
    for (int a = 0; a < D; ++a) pa[a] = 0.0f;
    float dadj = 0.0f;
    float madj_k[D * D], rda_k[D];
    if (P.state_grad && P.hybrid)
#pragma unroll
        for (int k = 0; k < D * D; ++k) madj_k[k] = A.madj[(uint64_t)s * 9 + k];
    if (P.density_grad)
#pragma unroll
        for (int a = 0; a < D; ++a) rda_k[a] = A.rda[(uint64_t)s * 4 + a];
    const float* rg_k = A.rga + (uint64_t)s * P.SS * D;
    float pi[3];
    int ci[3];
    load_rec<D>(A.srec, A.scoord, s, pi, ci);
    walk_neighbors<D>(P.g, b, pi, ci, A.bo, A.srec, A.scoord, [&](uint32_t j, const float* d, float r2) {
        const bool self = j == s;
        float dn[D];  // the pair's delta seen from j
#pragma unroll
        for (int a = 0; a < D; ++a) dn[a] = -d[a];
        const float rho_j = A.sdens[j];
        const float vol_j = recip_finite(rho_j);
        float sj[kCpl], fbj[kCpl];
#pragma unroll
        for (int u = 0; u < kCpl; ++u) {
            sj[u] = rowlane ? A.sstate[(uint64_t)j * P.SS + c0 + u] : 0.0f;
            fbj[u] = c0 + u < (int)S ? A.sfb[(uint64_t)j * P.SS + c0 + u] : 0.0f;
        }
        // blurred state (adjoint.rs:138-166): k as the neighbour of idx = j ...
        const float kern = poly6(r2, P.g);
        const float w = kern * vol_k;
        float wadj = 0.0f, wk = 0.0f;
#pragma unroll
        for (int u = 0; u < kCpl; ++u) {
            if (c0 + u >= (int)S) continue;
            acc[u] += fbj[u] * w;
            wadj += fbj[u] * sk[u];
            wk += fbk[u] * sj[u];
        }
        wadj = group_sum<L>(wadj);
        wk = group_sum<L>(wk);
        float t[D];
        if (lead) {
            poly6_delta_adjoint<D>(dn, r2, P.g, wadj * vol_k, t);
#pragma unroll
            for (int a = 0; a < D; ++a) pa[a] += t[a];
            volume_density_adjoint(rho_k, wadj * kern, &dadj);
        }
        if (self) return;  // the self pair's other terms are zero
        if (lead) {  // ... and k as idx with neighbour j
            poly6_delta_adjoint<D>(d, r2, P.g, wk * vol_j, t);
#pragma unroll
            for (int a = 0; a < D; ++a) pa[a] -= t[a];
        }
        if (P.state_grad) {  // adjoint.rs:276-347
            const float* rg_j = A.rga + (uint64_t)j * P.SS * D;
            // spiky_gradient_kernel for the three coefficients, from one square root: seen from j
            // with k's volume (vg) and with 1 (ug), seen from k with j's volume (vgk)
            const SpikyPre qk = spiky_pre(r2, P.g, vol_k), qj = spiky_pre(r2, P.g, vol_j);
            const SpikyPre q1 = spiky_pre(r2, P.g, 1.0f);
            float vg[D], ug[D], vgk[D];
#pragma unroll
            for (int a = 0; a < D; ++a) {
                vg[a] = qk.scale * dn[a];
                ug[a] = q1.scale * dn[a];
                vgk[a] = qj.scale * d[a];
            }
            // The delta adjoint is linear in its input: each role sums its channels' gradient
            // adjoints (gj: k as the neighbour of idx = j, gk: k as idx) and applies it once.
            float gj[D], gk[D];
#pragma unroll
            for (int a = 0; a < D; ++a) {
                gj[a] = 0.0f;
                gk[a] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kCpl; ++u) {
                const int c = c0 + u;
                if (c >= (int)S) continue;
                float sc = rg_j[c * D] * vg[0];
#pragma unroll
                for (int a = 1; a < D; ++a) sc += rg_j[c * D + a] * vg[a];
                acc[u] += sc;
                const float diff = sk[u] - sj[u];
#pragma unroll
                for (int a = 0; a < D; ++a) gj[a] += rg_j[c * D + a] * diff;
                float sk2 = rg_k[c * D] * vgk[0];
#pragma unroll
                for (int a = 1; a < D; ++a) sk2 += rg_k[c * D + a] * vgk[a];
                acc[u] -= sk2;
                const float diffk = sj[u] - sk[u];
#pragma unroll
                for (int a = 0; a < D; ++a) gk[a] += rg_k[c * D + a] * diffk;
            }
#pragma unroll
            for (int a = 0; a < D; ++a) {
                gj[a] = group_sum<L>(gj[a]);
                gk[a] = group_sum<L>(gk[a]);
            }
            if (lead) {
                spiky_delta_adjoint_pre<D>(dn, qk, gj, t);
#pragma unroll
                for (int a = 0; a < D; ++a) pa[a] += t[a];
                float va = gj[0] * ug[0];
#pragma unroll
                for (int a = 1; a < D; ++a) va += gj[a] * ug[a];
                volume_density_adjoint(rho_k, va, &dadj);
                spiky_delta_adjoint_pre<D>(d, qj, gk, t);
#pragma unroll
                for (int a = 0; a < D; ++a) pa[a] -= t[a];
            }
            if (P.hybrid && lead) {
                const float* mj = A.madj + (uint64_t)j * 9;
                // k as the neighbour of idx = j
                float dda[D], gda[D];
#pragma unroll
                for (int a = 0; a < D; ++a) {
                    dda[a] = 0.0f;
                    gda[a] = 0.0f;
                }
#pragma unroll
                for (int r = 0; r < D; ++r)
#pragma unroll
                    for (int cc = 0; cc < D; ++cc) {
                        const float m = mj[r * D + cc];
                        dda[r] += m * vg[cc];
                        gda[cc] += m * dn[r];
                    }
                spiky_delta_adjoint_pre<D>(dn, qk, gda, t);
#pragma unroll
                for (int a = 0; a < D; ++a) pa[a] += dda[a] + t[a];
                float va = gda[0] * ug[0];
#pragma unroll
                for (int a = 1; a < D; ++a) va += gda[a] * ug[a];
                volume_density_adjoint(rho_k, va, &dadj);
                // k as idx with neighbour j
#pragma unroll
                for (int a = 0; a < D; ++a) {
                    dda[a] = 0.0f;
                    gda[a] = 0.0f;
                }
#pragma unroll
                for (int r = 0; r < D; ++r)
#pragma unroll
                    for (int cc = 0; cc < D; ++cc) {
                        const float m = madj_k[r * D + cc];
                        dda[r] += m * vgk[cc];
                        gda[cc] += m * d[r];
                    }
                spiky_delta_adjoint_pre<D>(d, qj, gda, t);
#pragma unroll
                for (int a = 0; a < D; ++a) pa[a] -= dda[a] + t[a];
            }
        }
        if (P.density_grad && lead) {  // adjoint.rs:390-396
            const SpikyPre q1 = spiky_pre(r2, P.g, 1.0f);
            float rj[D];
#pragma unroll
            for (int a = 0; a < D; ++a) rj[a] = A.rda[(uint64_t)j * 4 + a];
            spiky_delta_adjoint_pre<D>(dn, q1, rj, t);
#pragma unroll
            for (int a = 0; a < D; ++a) pa[a] += t[a];
            spiky_delta_adjoint_pre<D>(d, q1, rda_k, t);
#pragma unroll
            for (int a = 0; a < D; ++a) pa[a] -= t[a];
        }
    });
#pragma unroll
    for (int a = 0; a < D; ++a) pa[a] = group_sum<L>(pa[a]);
    dadj = group_sum<L>(dadj);
    if (P.position_features) {  // adjoint.rs:118-122
        const uint32_t off = P.F - D;
#pragma unroll
        for (int a = 0; a < D; ++a) pa[a] += fa[off + a];
    }
#pragma unroll
    for (int u = 0; u < kCpl; ++u)
        if (c0 + u < (int)S) A.state_adj[pk * S + c0 + u] = acc[u];
    if (lead) {
        A.ppos[s] = make_float4(pa[0], D > 1 ? pa[1] : 0.0f, D > 2 ? pa[D > 2 ? 2 : 0] : 0.0f, 0.0f);
        A.dadj[s] = dadj;
    }
}

// accumulate_density_kernel_position_adjoint (adjoint.rs:399-418), gathered.
template <int D>
__global__ __launch_bounds__(256) void k_adj_density_kernel(StepParams P, AdjointArgs A) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= P.T) return;
    const uint32_t b = s / P.N;
    const uint64_t pk = (uint64_t)b * P.N + A.perm[s];
    const float4 p0 = A.ppos[s];
    float pa[3] = {p0.x, p0.y, p0.z};
    const float adj_k = A.dadj[s];
    float pi[3];
    int ci[3];
    load_rec<D>(A.srec, A.scoord, s, pi, ci);
    walk_neighbors<D>(P.g, b, pi, ci, A.bo, A.srec, A.scoord, [&](uint32_t j, const float* d, float r2) {
        if (j == s) return;  // delta 0: no term
        float dn[D], t[D];
#pragma unroll
        for (int a = 0; a < D; ++a) dn[a] = -d[a];
        poly6_delta_adjoint<D>(dn, r2, P.g, A.dadj[j], t);  // k as the neighbour of idx = j
#pragma unroll
        for (int a = 0; a < D; ++a) pa[a] += t[a];
        poly6_delta_adjoint<D>(d, r2, P.g, adj_k, t);  // k as idx
#pragma unroll
        for (int a = 0; a < D; ++a) pa[a] -= t[a];
    });
    A.pos_adj[pk] = make_float4(pa[0], pa[1], D == 3 ? pa[2] : 0.0f, 0.0f);
}

template <int D, int SM>
static hipError_t launch_adjoint_t(const StepParams& p, const AdjointArgs& a, hipStream_t stream) {
    const dim3 grid((p.T + 255) / 256), block(256);
    const dim3 grid_l((uint32_t)(((uint64_t)p.T * (SM / kCpl) + 255) / 256));
    hipLaunchKernelGGL(k_adj_density<D>, grid, block, 0, stream, p, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_adj_prep<D, SM>), grid_l, block, 0, stream, p, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((k_adj_gather<D, SM>), grid_l, block, 0, stream, p, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_adj_density_kernel<D>, grid, block, 0, stream, p, a);
    return hipGetLastError();
}

hipError_t launch_perceive_adjoint(const StepParams& p, Workspace& ws, AdjointWorkspace& aw, const float* fadj,
                                   float* state_adj, float4* pos_adj, hipStream_t stream) {
    if (p.T == 0) return hipSuccess;
    const uint64_t T = p.T;
    if (T * (32 / kCpl) >= (1ull << 32)) return hipErrorInvalidValue;  // thread ids of the lane groups
    hipError_t e;
    if ((e = aw.sdens.reserve(T * 4)) != hipSuccess) return e;
    if ((e = aw.sfb.reserve(T * p.SS * 4)) != hipSuccess) return e;
    if ((e = aw.rga.reserve(T * p.SS * 3 * 4)) != hipSuccess) return e;
    if ((e = aw.madj.reserve(T * 9 * 4)) != hipSuccess) return e;
    if ((e = aw.rda.reserve(T * 4 * 4)) != hipSuccess) return e;
    if ((e = aw.dadj.reserve(T * 4)) != hipSuccess) return e;
    if ((e = aw.ppos.reserve(T * 16)) != hipSuccess) return e;
    AdjointArgs a{};
    a.srec = ws.srec.as<float4>();
    a.scoord = ws.scoord.as<int4>();
    a.bo = ws.bin_offsets.as<uint32_t>();
    a.perm = ws.perm.as<uint32_t>();
    a.sstate = ws.sstate.as<float>();
    a.fadj = fadj;
    a.sdens = aw.sdens.as<float>();
    a.sfb = aw.sfb.as<float>();
    a.rga = aw.rga.as<float>();
    a.madj = aw.madj.as<float>();
    a.rda = aw.rda.as<float>();
    a.dadj = aw.dadj.as<float>();
    a.ppos = aw.ppos.as<float4>();
    a.state_adj = state_adj;
    a.pos_adj = pos_adj;
    const bool d3 = p.g.dim == 3;
    if (p.SS <= 8) return d3 ? launch_adjoint_t<3, 8>(p, a, stream) : launch_adjoint_t<2, 8>(p, a, stream);
    if (p.SS <= 16) return d3 ? launch_adjoint_t<3, 16>(p, a, stream) : launch_adjoint_t<2, 16>(p, a, stream);
    return d3 ? launch_adjoint_t<3, 32>(p, a, stream) : launch_adjoint_t<2, 32>(p, a, stream);
}

void AdjointWorkspace::release() {
    for (DevBuf* b : {&sdens, &sfb, &rga, &madj, &rda, &dadj, &ppos}) b->release();
}

}  // namespace npa
