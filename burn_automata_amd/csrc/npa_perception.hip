// npa_perception.hip - SPH neighbour passes and the rollout update on gfx950.
//
// Work mapping: the hashgrid build splits every bin into runs of one true cell and emits work
// items of <= 64/L consecutive slots of a run; L lanes serve each target. Every per-target sum is
// taken in the reference's neighbour order (cells dz, dy, dx; slots ascending = particle index
// ascending), so the sums are bit-identical to the CPU path.
//
//   k_density    rho_i = sum_j W_poly6(r_ij^2)                          forward.rs:145-160
//   k_active     update-mask targets; masked-out particles get the Euler step's wrap/clamp only
//   k_perceive   second pass (blur, state gradient, density gradient, moment matrix)
//                forward.rs:162-382 -> moment correction, scaling, log-norm
//                normalize.rs:5-118 -> feature row                     forward.rs:100-133
//   k_mlp_euler  update MLP model.rs:900-940 -> motion scaling model.rs:867-898 -> 3D gates
//                model.rs:806-837 -> masked Euler step.rs:4-55, written to the ping-pong
//                output in original particle order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "npa_internal.hpp"
#include "npa_neighbors.hpp"

// The build compiles this file once per part so the kernel instantiations compile in parallel:
// NPA_PART 0 holds the non-template kernels and the host launchers, 2 and 3 the second-pass and
// MLP kernels of that dimension (undefined: everything, one object).
#ifndef NPA_PART
#define NPA_PART -1
#endif
#define NPA_PART_MAIN (NPA_PART < 0 || NPA_PART == 0)
#define NPA_PART_DIM2 (NPA_PART < 0 || NPA_PART == 2)
#define NPA_PART_DIM3 (NPA_PART < 0 || NPA_PART == 3)

namespace npa {

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

// ------------------------------------------------------------------------------------------
// Neighbour passes over the split bins.
//
// A work item holds targets of one cell run, so their 3x3(x3) neighbour cells, the cells' runs and
// the loop bounds are wave-uniform (targets are still grouped by cell coordinates, which covers
// Grid mode and unsplit bins). A neighbour cell's run is walked in chunks of kChunk slots. Per
// target, candidates are visited in cell order (dz, dy, dx) and ascending slot order - ascending
// particle index within the cell, the reference's for_each_neighbor order - so every per-target
// sum is unchanged.
constexpr int kChunk = kNbChunk;

// Lanes per target for a sorted-state row width SM (each lane owns SM / L state channels).
template <int SM>
struct LanesPerTarget {
    static constexpr int L = SM >= 16 ? 4 : SM / 4;
    static constexpr int CPL = SM / L;
};

// Value of lane (group base + j) for groups of L consecutive lanes (L = 1, 2 or 4), via DPP.
// quad_perm reads a valid lane for every lane, so bound_ctrl (zero for an invalid source lane)
// never applies; with it set the compiler folds the permutation into the consuming VALU
// instruction (v_mul_f32_dpp, v_add_f32_dpp) instead of issuing a separate move.
template <int L, int J>
__device__ __forceinline__ float group_bcast(float v) {
    if constexpr (L == 1) {
        return v;
    } else if constexpr (L == 2) {
        constexpr int c = J == 0 ? (0 | (0 << 2) | (2 << 4) | (2 << 6)) : (1 | (1 << 2) | (3 << 4) | (3 << 6));
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), c, 0xf, 0xf, true));
    } else {
        constexpr int c = J | (J << 2) | (J << 4) | (J << 6);
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), c, 0xf, 0xf, true));
    }
}

// Value of lane (quad base + j) for a lane index j known only at compile time after unrolling.
template <int L>
__device__ __forceinline__ int group_bcast_k(int v, int j) {
    switch (j) {
        case 0: return __float_as_int(group_bcast<L, 0>(__int_as_float(v)));
        case 1: return __float_as_int(group_bcast<L, 1>(__int_as_float(v)));
        case 2: return __float_as_int(group_bcast<L, 2>(__int_as_float(v)));
        default: return __float_as_int(group_bcast<L, 3>(__int_as_float(v)));
    }
}

// OR of a 64-bit value over each group of L consecutive lanes (L = 1, 2 or 4), via DPP.
template <int L>
__device__ __forceinline__ uint64_t group_or(uint64_t m) {
    if constexpr (L == 1) return m;
    uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
    constexpr int swap1 = 1 | (0 << 2) | (3 << 4) | (2 << 6);  // quad_perm [1,0,3,2]
    lo |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, swap1, 0xf, 0xf, true);
    hi |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, swap1, 0xf, 0xf, true);
    if constexpr (L == 4) {
        constexpr int swap2 = 2 | (3 << 2) | (0 << 4) | (1 << 6);  // quad_perm [2,3,0,1]
        lo |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, swap2, 0xf, 0xf, true);
        hi |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, swap2, 0xf, 0xf, true);
    }
    return ((uint64_t)hi << 32) | lo;
}

template <int L>
__device__ __forceinline__ float ordered_group_sum(float acc, float v) {
    // acc + v(lane 0) + v(lane 1) + ... in lane order: candidate order within the round
    acc += group_bcast<L, 0>(v);
    if constexpr (L >= 2) acc += group_bcast<L, 1>(v);
    if constexpr (L >= 4) {
        acc += group_bcast<L, 2>(v);
        acc += group_bcast<L, 3>(v);
    }
    return acc;
}

// Orders this wave's LDS accesses before and after the call (the wave's lanes exchange data).
__device__ __forceinline__ void lds_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// density  forward.rs:145-160: rho_i = sum_j W_poly6(r_ij^2), four lanes per target. A work item
// holds up to 16 consecutive slots of one cell run, so its targets share their 3^D neighbour cells
// and walk the same candidates in the same order (cells dz, dy, dx; slots ascending). Lane q of a
// target tests candidates q, q + 4, ... of each chunk (<= 64 consecutive slots of a neighbour run)
// - in 2D read from LDS, where the wave's lanes put the chunk's 64 records with one load each, so
// a chunk costs one memory round trip instead of one per batch of four rounds (C2: 34 -> 29 us) -
// and every lane rebuilds the target's running sum in candidate order from the four lanes' terms
// with DPP broadcasts folded into the adds; a rejected candidate adds +0.0, which leaves the sum
// unchanged (it starts at +0.0 and never holds -0.0). Each round's accept bits come from one
// ballot. The targets of an unsplit bin (more cells than its directory holds) may lie in different
// cells: the item's coordinate groups then walk in turn.
// For the update-mask targets the accepted candidates are recorded for the second pass, which needs
// exactly the same set in the same order: per chunk (in visit order) its first slot and 64-bit
// accept mask at [row * max_chunks(D) + chunk] for the first max_chunks(D) chunks, and the chunk
// count at nb_count[row].
template <int D>
__global__ __launch_bounds__(256) void k_density_q(StepParams P, const float4* __restrict__ srec,
                                                   const int4* __restrict__ scoord,
                                                   const uint32_t* __restrict__ bo,
                                                   const uint32_t* __restrict__ perm,
                                                   const uint32_t* __restrict__ row_of,
                                                   const uint2* __restrict__ wl,
                                                   const uint32_t* __restrict__ wl_count,
                                                   float4* __restrict__ svol, float* __restrict__ density_out,
                                                   uint32_t* __restrict__ nb_base, uint64_t* __restrict__ nb_mask,
                                                   uint32_t* __restrict__ nb_count) {
    constexpr uint32_t MAXC = max_chunks(D);
    // 2D: each chunk's records are loaded once, one per lane, and the rounds read them from LDS
    constexpr bool kStage = D == 2;
    __shared__ float4 staged[kStage ? 4 : 1][64];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t t = lane >> 2, q = lane & 3;
    float4* stg = staged[kStage ? threadIdx.x >> 6 : 0];  // this wave's chunk, record k at [k]
    const uint32_t items = *wl_count;
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    for (uint32_t it = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); it < items; it += nwaves) {
        const uint2 item = wl[it];
        const bool active = t < item.y;
        const uint32_t s = item.x + (active ? t : 0u);
        const uint32_t b = item.x / P.N;
        float pi[3];
        int ci[3];
        load_rec<D>(srec, scoord, s, pi, ci);
        const uint32_t row = active ? row_of[s] : ~0u;
        const bool record = row != ~0u;
        float rho = 0.0f;
        uint32_t nch = 0;
        const uint64_t act_all = __ballot(active);
        uint64_t pending = act_all;
        while (pending) {
            const int leader = __ffsll((unsigned long long)pending) - 1;
            const int l0 = readlane_i(ci[0], leader), l1 = readlane_i(ci[1], leader);
            const int l2 = D == 3 ? readlane_i(ci[2], leader) : 0;
            const bool same = active && ci[0] == l0 && ci[1] == l1 && (D == 2 || ci[2] == l2);
            const uint64_t group = __ballot(same) & pending;
            pending &= ~group;
            const bool in_group = (group >> lane) & 1ull;
            const bool all_in = group == act_all && P.g.k6 <= 3.4028235e38f;  // the rounds' fast form
            uint32_t gch = 0;  // chunk index within the group's visit order (wave-uniform)
            uint32_t nb_beg, nb_end;
            bool nb_filter, nb_found;
            neighbor_runs<D>(P, bo, b, l0, l1, l2, lane, nb_beg, nb_end, nb_filter, nb_found);
            for (uint64_t cells = __ballot(nb_found); cells; cells &= cells - 1) {
                const int nk = __ffsll((unsigned long long)cells) - 1;  // ascending = visit order
                const int64_t n0 = (int64_t)l0 + nk % 3 - 1, n1 = (int64_t)l1 + (nk / 3) % 3 - 1;
                const int64_t n2 = D == 3 ? (int64_t)l2 + nk / 9 - 1 : 0;
                const uint32_t beg = (uint32_t)readlane_i((int)nb_beg, nk);
                const uint32_t end = (uint32_t)readlane_i((int)nb_end, nk);
                const bool filter = readlane_i((int)nb_filter, nk) != 0;
                for (uint32_t base = beg; base < end; base += kChunk, ++gch) {
                    const uint32_t m = end - base < (uint32_t)kChunk ? end - base : (uint32_t)kChunk;
                    const float4* cand = srec + base;
                    uint32_t mk[2] = {0u, 0u};  // accept mask, candidates 0-31 and 32-63
                    if constexpr (kStage) {
                        // lane k: record k (k < 64: past the run are other runs' records or the
                        // records' 64-slot padding); a slot past the run gets x = +inf, which no
                        // target is near, so no form of the rounds accepts it
                        float4 rc;
                        if (!filter) {
                            const float2 v = *reinterpret_cast<const float2*>(cand + lane);
                            rc = make_float4(v.x, v.y, 0.0f, 0.0f);
                        } else {
                            rc = cand[lane];
                        }
                        if (lane >= m) rc.x = __builtin_inff();
                        lds_wave_sync();  // the previous chunk's reads are done
                        stg[lane] = rc;
                        lds_wave_sync();
                    }
                    // FILT: an unsplit bin's candidates are tested for the cell; PER: periodic deltas;
                    // FAST: the group is every active target of the item (one cell: any item of a
                    // split bin) and the poly6 constant is finite - no lane masks in the rounds
                    auto walk = [&](auto FILT, auto PER, auto FAST) {
                        constexpr bool filt = decltype(FILT)::value, per = decltype(PER)::value;
                        constexpr bool fast = decltype(FAST)::value;
                        constexpr bool xy = D == 2 && !filt;  // only the position is read
                        // k < 64: slots past the run are other runs' records or the records'
                        // 64-slot padding, loaded and never accepted (k >= m fails `ok`; the fast
                        // form moves their x to +inf, which no target is near)
                        auto load = [&](uint32_t k) {
                            const float4* src = kStage ? stg : cand;
                            if constexpr (xy) {
                                const float2 v = *reinterpret_cast<const float2*>(src + k);
                                return make_float4(v.x, v.y, 0.0f, 0.0f);
                            } else {
                                return src[k];
                            }
                        };
                        auto test = [&](uint32_t r, const float4 rc) {  // round r: candidate 4 r + q
                            auto delta = [&](float a, float bj, int ax) {  // neighbor_delta hashgrid.rs:165-181
                                const float v = bj - a;
                                if constexpr (!per) return v;
                                const float up = v - P.g.extent[ax], dn = v + P.g.extent[ax];
                                return v > P.g.half[ax] ? up : (v < -P.g.half[ax] ? dn : v);
                            };
                            const float d0 = delta(pi[0], rc.x, 0);
                            const float d1 = delta(pi[1], rc.y, 1);
                            float r2 = d0 * d0;
                            r2 += d1 * d1;
                            if constexpr (D == 3) {
                                const float d2 = delta(pi[2], rc.z, 2);
                                r2 += d2 * d2;
                            }
                            const bool near = r2 < P.g.eps2;
                            if constexpr (fast) {
                                // a rejected candidate's term is +0.0 from x = max(eps^2 - r^2, +0.0)
                                // (r^2 >= eps^2, +inf or NaN); an accepted one has x > 0 and
                                // poly6's operations, so the sum is the masked form's
                                const float x = fmaxf(P.g.eps2 - r2, 0.0f);
                                rho = ordered_group_sum<4>(rho, P.g.k6 * x * x * x);
                                return (uint64_t)__builtin_amdgcn_ballot_w64(near);
                            }
                            const uint32_t k = 4 * r + q;
                            bool ok = in_group & (k < m);
                            if constexpr (filt) {
                                if constexpr (D == 2) {
                                    ok = ok & ((int64_t)__float_as_int(rc.z) == n0) & ((int64_t)__float_as_int(rc.w) == n1);
                                } else {
                                    const int4 cc = scoord[base + k];
                                    ok = ok & ((int64_t)cc.x == n0) & ((int64_t)cc.y == n1) & ((int64_t)cc.z == n2);
                                }
                            }
                            const bool acc_ok = ok & near;
                            // the accept bits straight from the two compare masks
                            const uint64_t bal = __builtin_amdgcn_ballot_w64(near) & __builtin_amdgcn_ballot_w64(ok);
                            rho = ordered_group_sum<4>(rho, acc_ok ? poly6(r2, P.g) : 0.0f);
                            return bal;
                        };
                        const uint32_t rounds = (m + 3) / 4;
                        // four batches of four rounds (candidates 16 j .. 16 j + 15), each batch's
                        // loads issued together; batch j fills bits 16 j .. of the mask, four per
                        // round: this target's four lanes of the round's ballot
#pragma unroll
                        for (uint32_t j = 0; j < 4; ++j) {
                            if (4 * j >= rounds) break;
                            float4 ra[4];
#pragma unroll
                            for (int u = 0; u < 4; ++u) ra[u] = load(16 * j + 4 * u + q);
                            if constexpr (fast && !kStage) {
                                if (16 * j + 16 > m) {  // the batch that reaches past the run
#pragma unroll
                                    for (int u = 0; u < 4; ++u)
                                        if (16 * j + 4 * u + q >= m) ra[u].x = __builtin_inff();
                                }
                            }
                            uint32_t bits = 0;
#pragma unroll
                            for (uint32_t u = 0; u < 4; ++u) {
                                if (4 * j + u < rounds) {
                                    const uint64_t bal = test(4 * j + u, ra[u]);
                                    bits |= ((uint32_t)(bal >> (lane & ~3u)) & 0xfu) << (4 * u);
                                }
                            }
                            mk[j >> 1] |= bits << (16 * (j & 1));
                        }
                    };
                    const bool periodic = P.g.boundary == 0;
                    using T_ = std::true_type;
                    using F_ = std::false_type;
                    if (filter) {
                        if (periodic) walk(T_{}, T_{}, F_{});
                        else walk(T_{}, F_{}, F_{});
                    } else if (all_in) {
                        if (periodic) walk(F_{}, T_{}, T_{});
                        else walk(F_{}, F_{}, T_{});
                    } else {
                        if (periodic) walk(F_{}, T_{}, F_{});
                        else walk(F_{}, F_{}, F_{});
                    }
                    if (in_group && q == 0 && record && gch < MAXC) {
                        nb_base[(uint64_t)row * MAXC + gch] = base;
                        nb_mask[(uint64_t)row * MAXC + gch] = ((uint64_t)mk[1] << 32) | mk[0];
                    }
                }
            }
            if (in_group) nch = gch;
        }
        if (active && q == 0) {
            svol[s] = make_float4(pi[0], pi[1], pi[2], recip_finite(rho));
            if (record) nb_count[row] = nch;
            if (density_out) density_out[b * P.N + perm[s]] = rho;
        }
    }
}

// The density pass for sparse 2D grids, four lanes per target and sixteen consecutive slots per wave:
// writes exactly what k_density_q writes (the same sum in the same order, the same chunk records),
// with the lanes of a target sharing its own neighbour runs instead of a wave sharing one cell's.
//   lookup: lane q of a target looks up its neighbour cells k = q, q + 4, q + 8 (visit order
//     k = (dy + 1) * 3 + (dx + 1)); the runs' starts, lengths and cell filters are broadcast within
//     the quad, and every lane holds the visit-order stream of the target's candidates: candidate
//     j lies in the last run k with P_k <= j (P: exclusive prefix of the run lengths) at slot
//     j + (start_k - P_k);
//   rounds: lane q tests candidate 4 r + q of the stream in round r (four rounds' records loaded
//     together), and every lane rebuilds the running sum in candidate order from the quad's four
//     terms (a rejected or missing candidate adds +0.0, which leaves the sum unchanged);
//   records (update-mask targets): the quad's accept nibbles, eight rounds per word, go to an LDS
//     bit stream of the first kStreamBits candidates (enough for every recorded chunk: max_chunks
//     of 64 candidates); afterwards the owner lane of run k writes each of the run's 64-slot chunks'
//     first slot and mask (bits [P_k + 64 c, ...) of the stream) for the first max_chunks chunks,
//     and nb_count = the target's chunk count, as the chunk loop of k_density_q counts them.
constexpr uint32_t kStreamWords = 24 * 64 / 32;  // max_chunks(2) chunks of 64 candidates

template <int D>
__global__ __launch_bounds__(256) void k_density_lanes(StepParams P, const float4* __restrict__ srec,
                                                       const uint32_t* __restrict__ bo,
                                                       const uint32_t* __restrict__ perm,
                                                       const uint32_t* __restrict__ row_of,
                                                       float4* __restrict__ svol, float* __restrict__ density_out,
                                                       uint32_t* __restrict__ nb_base, uint64_t* __restrict__ nb_mask,
                                                       uint32_t* __restrict__ nb_count) {
    static_assert(D == 2, "the four-lane sparse pass serves 2D grids (nine neighbour cells)");
    constexpr uint32_t MAXC = max_chunks(D);
    static_assert(MAXC * 64 == kStreamWords * 32, "the stream holds every recorded chunk");
    __shared__ uint32_t stream_lds[4][16][kStreamWords + 1];
    const uint32_t lane = threadIdx.x & 63, t = lane >> 2, q = lane & 3;
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    uint32_t* stream = stream_lds[threadIdx.x >> 6][t];
    const uint32_t s_raw = wave * 16 + t;
    if (wave * 16 >= P.T) return;  // (wave-uniform)
    const bool active = s_raw < P.T;
    const uint32_t s = active ? s_raw : P.T - 1;
    const uint32_t b = s / P.N;
    float pi[3];
    int ci[3];
    load_rec<D>(srec, nullptr, s, pi, ci);
    const uint32_t row = active ? row_of[s] : ~0u;
    const bool record = row != ~0u;
    // ---- lookup: lane q, cells q, q + 4, q + 8
    uint32_t obeg[3], olen[3];
    bool ofilt[3];
    {
        int64_t nc[3][3];
        bool want[3];
        uint32_t oend[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const uint32_t k = q + 4 * u;
            want[u] = k < 9 && active;
            nc[u][0] = (int64_t)ci[0] + (int)(k % 3) - 1;
            nc[u][1] = (int64_t)ci[1] + (int)(k / 3) - 1;
            nc[u][2] = 0;
        }
        cell_ranges<3>(P, bo, b, nc, want, obeg, oend, ofilt);
#pragma unroll
        for (int u = 0; u < 3; ++u) olen[u] = oend[u] - obeg[u];
    }
    // every run in every lane of the quad (run k lives in lane k % 4, register k / 4)
    uint32_t rbeg[9], rlen[9], rfilt = 0;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        rbeg[k] = (uint32_t)group_bcast_k<4>((int)obeg[k / 4], k % 4);
        rlen[k] = (uint32_t)group_bcast_k<4>((int)olen[k / 4], k % 4);
        rfilt |= ((uint32_t)group_bcast_k<4>((int)ofilt[k / 4], k % 4) & 1u) << k;
    }
    uint32_t pre[9], total = 0;
    int dlt[9];  // slot - stream position within run k
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        pre[k] = total;
        dlt[k] = (int)rbeg[k] - (int)total;
        total += rlen[k];
    }
    uint32_t rounds = (total + 3) / 4;
    rounds = wave_max_u32(rounds);
    const bool any_filter = __ballot(rfilt != 0) != 0ull;
    const float eps2 = P.g.eps2, k6 = P.g.k6;
    const bool periodic = P.g.boundary == 0;
    float rho = 0.0f;
    uint32_t word = 0;  // accept nibbles of eight rounds (candidates 32 w .. 32 w + 31)
    auto candidate = [&](uint32_t j, uint32_t& slot, int& kk) {  // run of stream position j, and its slot
        int d = dlt[0];
        kk = 0;
#pragma unroll
        for (int k = 1; k < 9; ++k) {
            const bool in = j >= pre[k];
            d = in ? dlt[k] : d;
            kk = in ? k : kk;
        }
        slot = (uint32_t)((int)j + d);
    };
    for (uint32_t r0 = 0; r0 < rounds; r0 += 4) {
        float4 rc[4];
        bool ok[4];
        int kr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t j = 4 * (r0 + u) + q;
            uint32_t slot;
            candidate(j, slot, kr[u]);
            ok[u] = active && j < total;
            rc[u] = srec[ok[u] ? slot : s];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (r0 + u >= rounds) break;
            bool acc_ok = ok[u];
            if (any_filter && ((rfilt >> kr[u]) & 1u)) {  // an unsplit bin: keep this cell's particles
                const int64_t n0 = (int64_t)ci[0] + kr[u] % 3 - 1, n1 = (int64_t)ci[1] + kr[u] / 3 - 1;
                acc_ok = acc_ok && (int64_t)__float_as_int(rc[u].z) == n0 && (int64_t)__float_as_int(rc[u].w) == n1;
            }
            float d0 = rc[u].x - pi[0], d1 = rc[u].y - pi[1];
            if (periodic) {
                d0 = delta_axis(pi[0], rc[u].x, 0, P.g);
                d1 = delta_axis(pi[1], rc[u].y, 1, P.g);
            }
            float r2 = d0 * d0;
            r2 += d1 * d1;
            const bool near = acc_ok && r2 < eps2;
            const float x = eps2 - r2;
            rho = ordered_group_sum<4>(rho, near ? k6 * x * x * x : 0.0f);  // smoothing_poly6_kernel
            const uint64_t bal = __builtin_amdgcn_ballot_w64(near);
            const uint32_t r = r0 + u;
            word |= ((uint32_t)(bal >> (lane & ~3u)) & 0xfu) << (4 * (r & 7u));
            if ((r & 7u) == 7u || r + 1 == rounds) {
                if (q == 0 && r / 8 < kStreamWords) stream[r / 8] = word;
                word = 0;
            }
        }
    }
    if (active && q == 0) {
        svol[s] = make_float4(pi[0], pi[1], pi[2], recip_finite(rho));
        if (density_out) density_out[b * P.N + perm[s]] = rho;
    }
    if (!__ballot(record)) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // chunks: run k holds ceil(len / 64), in visit order after the earlier runs' chunks
    uint32_t gch0[9], nch = 0;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        gch0[k] = nch;
        nch += (rlen[k] + 63) / 64;
    }
    if (!record) return;
    if (q == 0) nb_count[row] = nch;
    const uint32_t used = min((total + 31) / 32, kStreamWords);  // stream words written
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        const uint32_t k = q + 4 * u;
        if (k >= 9) break;
        for (uint32_t c = 0; 64 * c < rlen[k] && gch0[k] + c < MAXC; ++c) {
            const uint32_t a = pre[k] + 64 * c;  // stream bit of the chunk's first candidate
            const uint32_t L = min(64u, rlen[k] - 64 * c);
            const uint32_t w0 = a / 32, sh = a % 32;
            const uint64_t lo = (uint64_t)(w0 < used ? stream[w0] : 0u) | ((uint64_t)(w0 + 1 < used ? stream[w0 + 1] : 0u) << 32);
            const uint64_t hi = w0 + 2 < used ? stream[w0 + 2] : 0u;
            uint64_t m = sh ? (lo >> sh) | (hi << (64 - sh)) : lo;
            if (L < 64) m &= (1ull << L) - 1ull;
            nb_base[(uint64_t)row * MAXC + gch0[k] + c] = rbeg[k] + 64 * c;
            nb_mask[(uint64_t)row * MAXC + gch0[k] + c] = m;
        }
    }
}

// The same pass for sparse 3D grids (a surface in a 32^3 grid, say: a few particles per occupied
// cell), four lanes per target and sixteen consecutive slots per wave. A target's 27 neighbour runs
// go to a table in LDS (lane q looks up cells q, q + 4, ..., visit order k = (dz + 1) * 9 + (dy + 1)
// * 3 + (dx + 1)); the quad's first lane forms the runs' stream offsets, slot offsets and chunk
// numbers; in round r lane q tests stream position 4 r + q, finding its run by advancing through
// the table (positions only grow). Sums, the accept stream and the chunk records as in the 2D pass.
constexpr uint32_t kStreamWords3 = 48 * 64 / 32;  // max_chunks(3) chunks of 64 candidates

#if NPA_PART_MAIN
__global__ __launch_bounds__(256) void k_density_lanes3(StepParams P, const float4* __restrict__ srec,
                                                        const int4* __restrict__ scoord,
                                                        const uint32_t* __restrict__ bo,
                                                        const uint32_t* __restrict__ perm,
                                                        const uint32_t* __restrict__ row_of,
                                                        float4* __restrict__ svol, float* __restrict__ density_out,
                                                        uint32_t* __restrict__ nb_base, uint64_t* __restrict__ nb_mask,
                                                        uint32_t* __restrict__ nb_count) {
    constexpr int D = 3;
    constexpr uint32_t MAXC = max_chunks(D);
    static_assert(MAXC * 64 == kStreamWords3 * 32, "the stream holds every recorded chunk");
    struct Runs {
        uint32_t pre[28];  // stream position of run k's first candidate; pre[27] = the total
        uint32_t beg[27];  // run k's first slot
        uint32_t gch[28];  // run k's first chunk number; gch[27] = the chunk count
        uint32_t filt;     // runs of unsplit bins (cell filter)
    };
    __shared__ Runs runs_lds[4][16];
    __shared__ uint32_t stream_lds[4][16][kStreamWords3 + 1];
    const uint32_t lane = threadIdx.x & 63, t = lane >> 2, q = lane & 3;
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    Runs& R = runs_lds[threadIdx.x >> 6][t];
    uint32_t* stream = stream_lds[threadIdx.x >> 6][t];
    const uint32_t s_raw = wave * 16 + t;
    if (wave * 16 >= P.T) return;  // (wave-uniform)
    const bool active = s_raw < P.T;
    const uint32_t s = active ? s_raw : P.T - 1;
    const uint32_t b = s / P.N;
    float pi[3];
    int ci[3];
    load_rec<D>(srec, scoord, s, pi, ci);
    const uint32_t row = active ? row_of[s] : ~0u;
    const bool record = row != ~0u;
    // ---- lookup: lane q, cells q, q + 4, ... (lengths to pre[], starts to beg[], filters by bit)
    uint32_t fbits = 0;
    for (uint32_t k = q; k < 27; k += 4) {
        uint32_t beg = 0, end = 0;
        bool filt = false;
        if (active && !cell_range(P, bo, b, (int64_t)ci[0] + (int)(k % 3) - 1, (int64_t)ci[1] + (int)((k / 3) % 3) - 1,
                                  (int64_t)ci[2] + (int)(k / 9) - 1, beg, end, filt)) {
            beg = end = 0;
            filt = false;
        }
        R.pre[k] = end - beg;
        R.beg[k] = beg;
        fbits |= (filt ? 1u : 0u) << k;
    }
    fbits |= (uint32_t)group_bcast_k<4>((int)fbits, 1) | (uint32_t)group_bcast_k<4>((int)fbits, 2) |
             (uint32_t)group_bcast_k<4>((int)fbits, 3) | (uint32_t)group_bcast_k<4>((int)fbits, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (q == 0) {  // lengths -> stream offsets and chunk numbers
        uint32_t run = 0, ch = 0;
        for (int k = 0; k < 27; ++k) {
            const uint32_t len = R.pre[k];
            R.pre[k] = run;
            R.gch[k] = ch;
            run += len;
            ch += (len + 63) / 64;
        }
        R.pre[27] = run;
        R.gch[27] = ch;
        R.filt = fbits;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t total = R.pre[27];
    uint32_t rounds = (total + 3) / 4;
    rounds = wave_max_u32(rounds);
    const bool any_filter = __ballot(fbits != 0) != 0ull;
    const float eps2 = P.g.eps2, k6 = P.g.k6;
    const bool periodic = P.g.boundary == 0;
    float rho = 0.0f;
    uint32_t word = 0;
    uint32_t kk = 0, knext = R.pre[1];  // the run of this lane's stream position, and where the next starts
    for (uint32_t r0 = 0; r0 < rounds; r0 += 4) {
        float4 rc[4];
        int4 cc[4];
        bool ok[4];
        uint32_t kr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t j = 4 * (r0 + u) + q;
            ok[u] = active && j < total;
            if (ok[u])
                while (j >= knext) {  // advance to the run holding position j (empty runs skipped)
                    ++kk;
                    knext = R.pre[kk + 1];
                }
            const uint32_t slot = ok[u] ? R.beg[kk] + (j - R.pre[kk]) : s;
            kr[u] = kk;
            rc[u] = srec[slot];
            cc[u] = any_filter ? scoord[slot] : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (r0 + u >= rounds) break;
            bool acc_ok = ok[u];
            if (any_filter && ((fbits >> kr[u]) & 1u)) {  // an unsplit bin: keep this cell's particles
                const int k = (int)kr[u];
                acc_ok = acc_ok && (int64_t)cc[u].x == (int64_t)ci[0] + k % 3 - 1 &&
                         (int64_t)cc[u].y == (int64_t)ci[1] + (k / 3) % 3 - 1 && (int64_t)cc[u].z == (int64_t)ci[2] + k / 9 - 1;
            }
            float d0 = rc[u].x - pi[0], d1 = rc[u].y - pi[1], d2 = rc[u].z - pi[2];
            if (periodic) {
                d0 = delta_axis(pi[0], rc[u].x, 0, P.g);
                d1 = delta_axis(pi[1], rc[u].y, 1, P.g);
                d2 = delta_axis(pi[2], rc[u].z, 2, P.g);
            }
            float r2 = d0 * d0;
            r2 += d1 * d1;
            r2 += d2 * d2;
            const bool near = acc_ok && r2 < eps2;
            const float x = eps2 - r2;
            rho = ordered_group_sum<4>(rho, near ? k6 * x * x * x : 0.0f);  // smoothing_poly6_kernel
            const uint64_t bal = __builtin_amdgcn_ballot_w64(near);
            const uint32_t r = r0 + u;
            word |= ((uint32_t)(bal >> (lane & ~3u)) & 0xfu) << (4 * (r & 7u));
            if ((r & 7u) == 7u || r + 1 == rounds) {
                if (q == 0 && r / 8 < kStreamWords3) stream[r / 8] = word;
                word = 0;
            }
        }
    }
    if (active && q == 0) {
        svol[s] = make_float4(pi[0], pi[1], pi[2], recip_finite(rho));
        if (density_out) density_out[b * P.N + perm[s]] = rho;
    }
    if (!__ballot(record)) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (!record) return;
    if (q == 0) nb_count[row] = R.gch[27];
    const uint32_t used = min((total + 31) / 32, kStreamWords3);
    for (uint32_t k = q; k < 27; k += 4) {
        const uint32_t len = R.pre[k + 1] - R.pre[k], g0 = R.gch[k];
        for (uint32_t c = 0; 64 * c < len && g0 + c < MAXC; ++c) {
            const uint32_t a = R.pre[k] + 64 * c;  // stream bit of the chunk's first candidate
            const uint32_t L = min(64u, len - 64 * c);
            const uint32_t w0 = a / 32, sh = a % 32;
            const uint64_t lo = (uint64_t)(w0 < used ? stream[w0] : 0u) | ((uint64_t)(w0 + 1 < used ? stream[w0 + 1] : 0u) << 32);
            const uint64_t hi = w0 + 2 < used ? stream[w0 + 2] : 0u;
            uint64_t m = sh ? (lo >> sh) | (hi << (64 - sh)) : lo;
            if (L < 64) m &= (1ull << L) - 1ull;
            nb_base[(uint64_t)row * MAXC + g0 + c] = R.beg[k] + 64 * c;
            nb_mask[(uint64_t)row * MAXC + g0 + c] = m;
        }
    }
}

// The sparse pass with a 16-lane row per target (four targets per wave): a sparse grid (a surface in
// a 32^3 grid, say) gives each target few candidates (about 56 at C4) behind 3^D run look-ups, so
// the pass is set by its memory round trips, not by issue. Sixteen lanes per target look up the
// cells in at most two steps (lane q: cells q and q + 16), form the runs' stream offsets and chunk
// numbers with row scans, and test 16 candidates per round (lane q: stream position 16 r + q, four
// rounds' records loaded together), the running sum rebuilt in candidate order from the row's 16
// terms through DPP row_newbcast. Same sum, same order, same records as k_density_q.
template <int K>
__device__ __forceinline__ float row_lane(float v) {  // lane K of this lane's 16-lane row
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + K, 0xf, 0xf, false));
}

// OR over the 16 lanes of each row (quads, half rows, then the row's halves; DPP, no LDS trip).
__device__ __forceinline__ uint32_t row_or16(uint32_t v) {
    v |= dpp_or_identity<0xb1, 0xf>(0u, v);   // quad_perm [1,0,3,2]
    v |= dpp_or_identity<0x4e, 0xf>(0u, v);   // quad_perm [2,3,0,1]
    v |= dpp_or_identity<0x141, 0xf>(0u, v);  // row_half_mirror
    v |= dpp_or_identity<0x140, 0xf>(0u, v);  // row_mirror
    return v;
}
// Lane 15 of this lane's row (DPP row_newbcast:15).
__device__ __forceinline__ uint32_t row_last16(uint32_t v) { return dpp_or_identity<0x15f, 0xf>(0u, v); }

template <int D>
__global__ __launch_bounds__(256) void k_density_rows(StepParams P, const float4* __restrict__ srec,
                                                       const int4* __restrict__ scoord,
                                                       const uint32_t* __restrict__ bo,
                                                       const uint32_t* __restrict__ perm,
                                                       const uint32_t* __restrict__ row_of,
                                                       float4* __restrict__ svol, float* __restrict__ density_out,
                                                       uint32_t* __restrict__ nb_base, uint64_t* __restrict__ nb_mask,
                                                       uint32_t* __restrict__ nb_count) {
    constexpr uint32_t MAXC = max_chunks(D);
    constexpr int NC = D == 3 ? 27 : 9;  // neighbour cells
    constexpr uint32_t SW = D == 3 ? kStreamWords3 : kStreamWords;
    static_assert(MAXC * 64 == SW * 32, "the stream holds every recorded chunk");
    struct Runs {
        uint32_t pre[NC + 1];  // stream position of run k's first candidate; pre[NC] = the total
        uint32_t beg[NC];      // run k's first slot
        uint32_t gch[NC + 1];  // run k's first chunk number; gch[NC] = the chunk count
    };
    __shared__ Runs runs_lds[4][4];
    __shared__ uint32_t stream_lds[4][4][SW + 1];
    const uint32_t lane = threadIdx.x & 63, t = lane >> 4, q = lane & 15;
    const uint32_t wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    Runs& R = runs_lds[threadIdx.x >> 6][t];
    uint32_t* stream = stream_lds[threadIdx.x >> 6][t];
    const uint32_t s_raw = wave * 4 + t;
    if (wave * 4 >= P.T) return;  // (wave-uniform)
    const bool active = s_raw < P.T;
    const uint32_t s = active ? s_raw : P.T - 1;
    const uint32_t b = s / P.N;
    float pi[3];
    int ci[3];
    load_rec<D>(srec, scoord, s, pi, ci);
    const uint32_t row = active ? row_of[s] : ~0u;
    const bool record = row != ~0u;
    // ---- look-ups: lane q, cells q and q + 16 (visit order k = (dz + 1) * 9 + (dy + 1) * 3 + (dx + 1))
    uint32_t beg[2] = {0u, 0u}, len[2] = {0u, 0u}, fbits = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint32_t k = q + 16 * u;
        uint32_t bb = 0, ee = 0;
        bool filt = false;
        if (k < (uint32_t)NC && active &&
            cell_range(P, bo, b, (int64_t)ci[0] + (int)(k % 3) - 1, (int64_t)ci[1] + (int)((k / 3) % 3) - 1,
                       D == 3 ? (int64_t)ci[2] + (int)(k / 9) - 1 : 0, bb, ee, filt)) {
            beg[u] = bb;
            len[u] = ee - bb;
            fbits |= (filt ? 1u : 0u) << k;
        }
    }
    // the row's filter bits, stream offsets and chunk numbers (exclusive prefixes over k)
    fbits = row_or16(fbits);
    const uint32_t ch0 = (len[0] + 63) / 64, ch1 = (len[1] + 63) / 64;
    const uint32_t x0 = row_incl_add(len[0]), x1 = row_incl_add(len[1]);
    const uint32_t y0 = row_incl_add(ch0), y1 = row_incl_add(ch1);
    const uint32_t tot0 = row_last16(x0), tch0 = row_last16(y0);
    const uint32_t tot1 = row_last16(x1), tch1 = row_last16(y1);
    if (q < (uint32_t)NC) {
        R.pre[q] = x0 - len[0];
        R.beg[q] = beg[0];
        R.gch[q] = y0 - ch0;
    }
    if (q + 16 < (uint32_t)NC) {
        R.pre[q + 16] = tot0 + x1 - len[1];
        R.beg[q + 16] = beg[1];
        R.gch[q + 16] = tch0 + y1 - ch1;
    }
    if (q == 0) {
        R.pre[NC] = tot0 + tot1;
        R.gch[NC] = tch0 + tch1;
    }
    lds_wave_sync();
    const uint32_t total = tot0 + tot1;
    uint32_t rounds = (total + 15) / 16;
    rounds = wave_max_u32(rounds);
    const bool any_filter = __ballot(fbits != 0) != 0ull;
    const float eps2 = P.g.eps2, k6 = P.g.k6;
    const bool periodic = P.g.boundary == 0;
    float rho = 0.0f;
    uint32_t kk = 0, knext = R.pre[1];  // the run of this lane's stream position, and where the next starts
    for (uint32_t r0 = 0; r0 < rounds; r0 += 4) {
        float4 rc[4];
        int4 cc[4];
        bool ok[4];
        uint32_t kr[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t j = 16 * (r0 + u) + q;
            ok[u] = active && j < total;
            if (ok[u])
                while (j >= knext) {  // advance to the run holding position j (empty runs skipped)
                    ++kk;
                    knext = R.pre[kk + 1];
                }
            const uint32_t slot = ok[u] ? R.beg[kk] + (j - R.pre[kk]) : s;
            kr[u] = kk;
            rc[u] = srec[slot];
            cc[u] = D == 3 && any_filter ? scoord[slot] : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (r0 + u >= rounds) break;
            bool acc_ok = ok[u];
            if (any_filter && ((fbits >> kr[u]) & 1u)) {  // an unsplit bin: keep this cell's particles
                const int k = (int)kr[u];
                if constexpr (D == 3)
                    acc_ok = acc_ok && (int64_t)cc[u].x == (int64_t)ci[0] + k % 3 - 1 &&
                             (int64_t)cc[u].y == (int64_t)ci[1] + (k / 3) % 3 - 1 &&
                             (int64_t)cc[u].z == (int64_t)ci[2] + k / 9 - 1;
                else  // 2D records carry the cell coordinates' bits in z and w
                    acc_ok = acc_ok && (int64_t)__float_as_int(rc[u].z) == (int64_t)ci[0] + k % 3 - 1 &&
                             (int64_t)__float_as_int(rc[u].w) == (int64_t)ci[1] + k / 3 - 1;
            }
            float d0 = rc[u].x - pi[0], d1 = rc[u].y - pi[1], d2 = D == 3 ? rc[u].z - pi[2] : 0.0f;
            if (periodic) {
                d0 = delta_axis(pi[0], rc[u].x, 0, P.g);
                d1 = delta_axis(pi[1], rc[u].y, 1, P.g);
                if constexpr (D == 3) d2 = delta_axis(pi[2], rc[u].z, 2, P.g);
            }
            float r2 = d0 * d0;
            r2 += d1 * d1;
            if constexpr (D == 3) r2 += d2 * d2;
            const bool near = acc_ok && r2 < eps2;
            const float x = eps2 - r2;
            const float term = near ? k6 * x * x * x : 0.0f;  // smoothing_poly6_kernel
            // the running sum in candidate order: lane 0's term first (a rejected one adds +0.0)
            rho += row_lane<0>(term);
            rho += row_lane<1>(term);
            rho += row_lane<2>(term);
            rho += row_lane<3>(term);
            rho += row_lane<4>(term);
            rho += row_lane<5>(term);
            rho += row_lane<6>(term);
            rho += row_lane<7>(term);
            rho += row_lane<8>(term);
            rho += row_lane<9>(term);
            rho += row_lane<10>(term);
            rho += row_lane<11>(term);
            rho += row_lane<12>(term);
            rho += row_lane<13>(term);
            rho += row_lane<14>(term);
            rho += row_lane<15>(term);
            const uint64_t bal = __builtin_amdgcn_ballot_w64(near);
            const uint32_t r = r0 + u;
            // the target's 16 accept bits = stream bits 16 r .. 16 r + 15
            const uint32_t bits = (uint32_t)(bal >> (16 * t)) & 0xffffu;
            if (q == 0 && r / 2 < SW) {
                if ((r & 1u) == 0) stream[r / 2] = bits;
                else stream[r / 2] |= bits << 16;
            }
        }
    }
    if (active && q == 0) {
        svol[s] = make_float4(pi[0], pi[1], pi[2], recip_finite(rho));
        if (density_out) density_out[b * P.N + perm[s]] = rho;
    }
    if (!__ballot(record)) return;
    lds_wave_sync();
    if (!record) return;
    if (q == 0) nb_count[row] = R.gch[NC];
    const uint32_t used = min((total + 31) / 32, SW);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint32_t k = q + 16 * u;
        if (k >= (uint32_t)NC) break;
        const uint32_t rl = R.pre[k + 1] - R.pre[k], g0 = R.gch[k];
        for (uint32_t c = 0; 64 * c < rl && g0 + c < MAXC; ++c) {
            const uint32_t a = R.pre[k] + 64 * c;  // stream bit of the chunk's first candidate
            const uint32_t L = min(64u, rl - 64 * c);
            const uint32_t w0 = a / 32, sh = a % 32;
            const uint64_t lo = (uint64_t)(w0 < used ? stream[w0] : 0u) | ((uint64_t)(w0 + 1 < used ? stream[w0 + 1] : 0u) << 32);
            const uint64_t hi = w0 + 2 < used ? stream[w0 + 2] : 0u;
            uint64_t m = sh ? (lo >> sh) | (hi << (64 - sh)) : lo;
            if (L < 64) m &= (1ull << L) - 1ull;
            nb_base[(uint64_t)row * MAXC + g0 + c] = R.beg[k] + 64 * c;
            nb_mask[(uint64_t)row * MAXC + g0 + c] = m;
        }
    }
}
#endif  // NPA_PART_MAIN

// Per-wave accepted-neighbour lists of the second pass: the sorted slots of each target's accepted
// candidates, appended in visit order (cells dz, dy, dx; slots ascending), so walking a list front
// to back is the reference's neighbour order. kListBytes of LDS per wave for any targets-per-item.
constexpr int kListBytes = 12288;

template <int TPI>
struct PerceiveLists {
    static constexpr int CAP = kListBytes / (4 * TPI);
    uint32_t slot[CAP][TPI];
};

// Bits k of a 64-bit chunk mask with k % L == q.
template <int L>
__device__ __forceinline__ uint64_t residue_mask(uint32_t q) {
    if constexpr (L == 1) return ~0ull;
    else if constexpr (L == 2) return 0x5555555555555555ull << q;
    else return 0x1111111111111111ull << q;
}

// Second neighbour pass + normalisation + feature row, L lanes per target, each lane owning
// CPL = SM / L state channels.
// Phase A: the target's accepted candidates are appended to its list in LDS, chunk by chunk in
//   visit order, from the accept masks the density pass recorded (the same test on the same
//   candidates). A target with more chunks than were recorded makes the item test them here: for
//   each neighbour cell of the target's cell (reference order), the L lanes of a target test the
//   candidates round-robin straight from the sorted records and OR their accept masks.
// Phase B (when a list would overflow, and at the end): the lists are consumed in rounds of L
//   entries: lane q computes the pair scalars (poly6, volume, spiky gradients) of the round's
//   q-th entry, and every lane applies the round's entries in list order to its own channels,
//   with the scalars and the candidate slot broadcast inside the lane group and the candidate's
//   state channels read from the sorted state rows. Rounds span all of a target's neighbour
//   bins, so the targets of a wave stay busy for about the same number of rounds. Each round's
//   loads are issued two rounds before it is computed (three register sets).
// Padding entries (a short last round, a target with fewer entries than the wave's longest
// list) use the target itself with zero weights; the self pair's gradient terms and those of
// coincident particles are zero as well. Zero terms leave every sum unchanged: each sum starts
// at +0.0 and so never holds -0.0.
// MODE 0: padded feature rows, feature-major (features[k * T + s]) for the MLP kernel.
// MODE 1: the perceive_with_options outputs in original particle order.
// FL >= 0 fixes the option flags at compile time (bit 0 state gradient, bit 1 density gradient,
// bit 2 moment correction); FL < 0 reads them from P.
template <int D, int SM, int MODE, int FL>
__global__ __launch_bounds__(64) void k_perceive(StepParams P, const float4* __restrict__ srec,
                                                 const int4* __restrict__ scoord,
                                                 const float* __restrict__ sstate,
                                                 const float4* __restrict__ svol,
                                                 const uint32_t* __restrict__ bo,
                                                 const uint32_t* __restrict__ perm,
                                                 const uint32_t* __restrict__ act_rows,
                                                 const uint32_t* __restrict__ row_count,
                                                 const uint32_t* __restrict__ nb_base,
                                                 const uint64_t* __restrict__ nb_mask,
                                                 const uint32_t* __restrict__ nb_count,
                                                 float* __restrict__ sfeatures, StepIO io) {
    constexpr int L = LanesPerTarget<SM>::L;
    constexpr int CPL = LanesPerTarget<SM>::CPL;
    constexpr int TPI = 64 / L;
    constexpr uint32_t MAXC = max_chunks(D);
    using Lists = PerceiveLists<TPI>;
    constexpr uint32_t CAP = Lists::CAP;
    __shared__ Lists lists;
    const uint32_t lane = threadIdx.x;
    const uint32_t t = lane / L, q = lane % L;
    const uint32_t c0 = q * CPL;  // first channel of this lane
    const uint32_t nrows = *row_count;
    const uint32_t items = (nrows + TPI - 1) / TPI;  // TPI consecutive compact rows per wave
    const bool want_sg = FL >= 0 ? (FL & 1) != 0 : P.state_grad != 0;
    const bool want_dg = FL >= 0 ? (FL & 2) != 0 : P.density_grad != 0;
    const bool want_m = FL >= 0 ? (FL & 5) == 5 : (want_sg && P.hybrid);
    const bool branch_a = want_sg && want_dg;
    const uint64_t my_residue = residue_mask<L>(q);
    for (uint32_t it = blockIdx.x; it < items; it += gridDim.x) {
        const uint32_t row = it * TPI + t;  // compact feature row
        const bool active = row < nrows;
        const uint32_t s = act_rows[active ? row : it * TPI];
        const uint32_t b = s / P.N;
        float pi[3];
        int ci[3];
        load_rec<D>(srec, scoord, s, pi, ci);
        float si[CPL], blur[CPL], grad[CPL * D], dg[D], mom[D * D];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            si[c] = sstate[(uint64_t)s * SM + c0 + c];
            blur[c] = 0.0f;
        }
#pragma unroll
        for (int k = 0; k < CPL * D; ++k) grad[k] = 0.0f;
#pragma unroll
        for (int k = 0; k < D; ++k) dg[k] = 0.0f;
#pragma unroll
        for (int k = 0; k < D * D; ++k) mom[k] = 0.0f;

        uint32_t cnt = 0;      // entries in this target's list (same in the L lanes of a target)

        // Phase B over the current lists. Round r: lane q takes entry r * L + q of its target's list.
        // The loads of round r + 1 (the entry's record, volume and the round's state rows) are
        // issued before round r is computed, so their latency overlaps the arithmetic.
        struct Fetch {
            uint32_t slot;
            bool has;
            float4 rj;
            float vj;
            float sv[L][CPL];
        };
        // list entry of round r (index clamped: in bounds for any r)
        auto entry = [&](uint32_t r) {
            const uint32_t e = r * L + q;
            return lists.slot[e < CAP ? e : CAP - 1][t];
        };
        uint32_t next_en = 0;  // entry of the next round to fetch, read one fetch ahead
        auto fetch = [&](uint32_t r, Fetch& F) {
            const uint32_t e = r * L + q;
            F.has = active && e < cnt;
            const uint32_t en = next_en;
            next_en = entry(r + 1);  // LDS latency overlaps the next round
            F.slot = F.has ? en : s;  // a lane without an entry uses its target
            F.rj = svol[F.slot];  // position and volume of the candidate
            F.vj = F.rj.w;
            uint32_t rs[L];
            auto bslot = [&](auto J) {
                return (uint32_t)__float_as_int(group_bcast<L, decltype(J)::value>(__int_as_float((int)F.slot)));
            };
            rs[0] = bslot(std::integral_constant<int, 0>{});
            if constexpr (L >= 2) rs[1] = bslot(std::integral_constant<int, 1>{});
            if constexpr (L >= 4) {
                rs[2] = bslot(std::integral_constant<int, 2>{});
                rs[3] = bslot(std::integral_constant<int, 3>{});
            }
#pragma unroll
            for (int j = 0; j < L; ++j) {
                const float* rowp = sstate + (uint64_t)rs[j] * SM + c0;
                if constexpr (CPL % 4 == 0) {  // 16-byte aligned channel slices
                    const float4* row = reinterpret_cast<const float4*>(rowp);
#pragma unroll
                    for (int v = 0; v < CPL / 4; ++v) {
                        const float4 x = row[v];
                        F.sv[j][4 * v + 0] = x.x;
                        F.sv[j][4 * v + 1] = x.y;
                        F.sv[j][4 * v + 2] = x.z;
                        F.sv[j][4 * v + 3] = x.w;
                    }
                } else {  // CPL = 6 (SM = 24): 8-byte aligned slices
                    static_assert(CPL % 2 == 0, "channel slices are whole float2s");
                    const float2* row = reinterpret_cast<const float2*>(rowp);
#pragma unroll
                    for (int v = 0; v < CPL / 2; ++v) {
                        const float2 x = row[v];
                        F.sv[j][2 * v + 0] = x.x;
                        F.sv[j][2 * v + 1] = x.y;
                    }
                }
            }
        };
        auto compute = [&](const Fetch& F) {
            // pair scalars of this lane's entry, branch-free; a lane without an entry (or the
            // self pair / a coincident particle for the gradients) selects zeros
            const bool has = F.has;
            const float4 rj = F.rj;
            const float vj = F.vj;
            float d[3];
            d[0] = delta_axis(pi[0], rj.x, 0, P.g);
            d[1] = delta_axis(pi[1], rj.y, 1, P.g);
            d[2] = 0.0f;
            float r2 = d[0] * d[0];
            r2 += d[1] * d[1];
            if constexpr (D == 3) {
                d[2] = delta_axis(pi[2], rj.z, 2, P.g);
                r2 += d[2] * d[2];
            }
            const float smooth = has ? poly6(r2, P.g) : 0.0f;
            const float vol = has ? vj : 0.0f;
            const bool gok = has && F.slot != s && r2 > 0.0f;  // spiky_gradient_kernel kernels.rs:79-96
            const float rr = sqrtf(r2);
            const float tt = P.g.eps - rr;
            float vg[D], dgv[D];
#pragma unroll
            for (int a = 0; a < D; ++a) {
                vg[a] = 0.0f;
                dgv[a] = 0.0f;
            }
            if (want_dg) {
                const float mag = 1.0f * P.g.k5 * 3.0f * (tt * tt) / rr;
#pragma unroll
                for (int a = 0; a < D; ++a) dgv[a] = gok ? mag * d[a] : 0.0f;
            }
            if (want_sg) {
                const float mag = vj * P.g.k5 * 3.0f * (tt * tt) / rr;
#pragma unroll
                for (int a = 0; a < D; ++a) vg[a] = gok ? mag * d[a] : 0.0f;
            }
            const float w = smooth * vol;  // blur_state weight (density-grad-off branch)
            // moment terms delta[ra] * grad[ca] of this lane's entry, upper triangle (the only
            // entries safe_inverse_symmetric reads); the lanes then add the round's terms in order
            float mp[D * (D + 1) / 2];
            if (want_m) {
                int k = 0;
#pragma unroll
                for (int ra = 0; ra < D; ++ra)
#pragma unroll
                    for (int ca = ra; ca < D; ++ca) mp[k++] = d[ra] * vg[ca];
            }
            // the round's entries in list order
            auto round_step = [&](auto J) {
                constexpr int j = decltype(J)::value;
                if (branch_a) {  // second_pass_particle forward.rs:263-270
                    const float c_smooth = group_bcast<L, j>(smooth), c_vol = group_bcast<L, j>(vol);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) blur[c] += F.sv[j][c] * c_smooth * c_vol;
                } else {  // blur_state forward.rs:174-180
                    const float c_w = group_bcast<L, j>(w);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) blur[c] += F.sv[j][c] * c_w;
                }
                if (want_dg) {
#pragma unroll
                    for (int a = 0; a < D; ++a) dg[a] += group_bcast<L, j>(dgv[a]);
                }
                if (want_sg) {
                    float c_vg[D];
#pragma unroll
                    for (int a = 0; a < D; ++a) c_vg[a] = group_bcast<L, j>(vg[a]);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const float diff = F.sv[j][c] - si[c];
#pragma unroll
                        for (int a = 0; a < D; ++a) grad[c * D + a] += diff * c_vg[a];
                    }
                    if (want_m) {
                        int k = 0;
#pragma unroll
                        for (int ra = 0; ra < D; ++ra)
#pragma unroll
                            for (int ca = ra; ca < D; ++ca) mom[ra * D + ca] += group_bcast<L, j>(mp[k++]);
                    }
                }
            };
            round_step(std::integral_constant<int, 0>{});
            if constexpr (L >= 2) round_step(std::integral_constant<int, 1>{});
            if constexpr (L >= 4) {
                round_step(std::integral_constant<int, 2>{});
                round_step(std::integral_constant<int, 3>{});
            }
        };
        auto flush = [&]() {
            __syncthreads();  // list writes of every lane are visible
            if (__ballot(active && 0u < cnt)) {
                // Rounds are fetched two ahead, unconditionally (past the end every lane loads its
                // own target's rows, unused), so no branch merges the load queues and each round
                // waits only for its own loads.
                Fetch A, B, C;
                next_en = entry(0);
                fetch(0, A);
                fetch(1, B);
                for (uint32_t r = 0;; r += 3) {
                    const bool m1 = __ballot(active && (r + 1) * L < cnt) != 0;
                    fetch(r + 2, C);
                    compute(A);
                    if (!m1) break;
                    const bool m2 = __ballot(active && (r + 2) * L < cnt) != 0;
                    fetch(r + 3, A);
                    compute(B);
                    if (!m2) break;
                    const bool m3 = __ballot(active && (r + 3) * L < cnt) != 0;
                    fetch(r + 4, B);
                    compute(C);
                    if (!m3) break;
                }
            }
            __syncthreads();  // every lane has read the lists before they are refilled
            cnt = 0;
        };

        // Phase A. The density pass recorded each target's accepted candidates per chunk, in visit
        // order; the lists are built from those masks (RB chunk records loaded per batch).
        const uint32_t nct = active ? nb_count[row] : 0u;
        const bool recorded = !__ballot(nct > MAXC);
        constexpr int RB = 2;  // chunk records loaded per batch
        for (uint32_t cb = 0; recorded && __ballot(cb < nct); cb += RB) {
            uint4 rc[RB];
#pragma unroll
            for (int u = 0; u < RB; ++u) {
                const uint32_t c = cb + (uint32_t)u;
                if (c < nct) {
                    const uint64_t mk = nb_mask[(uint64_t)row * MAXC + c];
                    rc[u] = make_uint4(nb_base[(uint64_t)row * MAXC + c], 0u, (uint32_t)mk, (uint32_t)(mk >> 32));
                } else {
                    rc[u] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
#pragma unroll
            for (int u = 0; u < RB; ++u) {
                const uint32_t c = cb + (uint32_t)u;
                const uint64_t acc = ((uint64_t)rc[u].w << 32) | rc[u].z;  // 0 past the target's chunks
                const uint32_t add = (uint32_t)__popcll(acc);
                if (__ballot(cnt + add > CAP)) flush();
                uint64_t mine = acc & my_residue;
                while (mine) {
                    const uint32_t k = (uint32_t)__builtin_ctzll(mine);
                    mine &= mine - 1;
                    const uint32_t pos = cnt + (uint32_t)__popcll(acc & ((1ull << k) - 1ull));
                    lists.slot[pos][t] = rc[u].x + k;
                }
                cnt += add;
            }
        }
        // Otherwise (a target with more chunks than were recorded): the coordinate groups of the
        // item, then each group's neighbour cells in order, testing the candidates here.
        uint64_t pending = recorded ? 0ull : __ballot(active);
        while (pending) {
            const int leader = __ffsll((unsigned long long)pending) - 1;
            const int l0 = readlane_i(ci[0], leader), l1 = readlane_i(ci[1], leader);
            const int l2 = D == 3 ? readlane_i(ci[2], leader) : 0;
            const uint32_t lb = (uint32_t)readlane_i((int)b, leader);
            const bool same = active && ci[0] == l0 && ci[1] == l1 && (D == 2 || ci[2] == l2) && b == lb;
            const uint64_t group = __ballot(same) & pending;
            pending &= ~group;
            const bool in_group = (group >> lane) & 1ull;
            uint32_t nb_beg, nb_end;
            bool nb_filter, nb_found;
            neighbor_runs<D>(P, bo, lb, l0, l1, l2, lane, nb_beg, nb_end, nb_filter, nb_found);
            for (uint64_t cells = __ballot(nb_found); cells; cells &= cells - 1) {
                const int nk = __ffsll((unsigned long long)cells) - 1;  // ascending = visit order
                const int64_t n0 = (int64_t)l0 + nk % 3 - 1, n1 = (int64_t)l1 + (nk / 3) % 3 - 1;
                const int64_t n2 = D == 3 ? (int64_t)l2 + nk / 9 - 1 : 0;
                const uint32_t beg = (uint32_t)readlane_i((int)nb_beg, nk);
                const uint32_t end = (uint32_t)readlane_i((int)nb_end, nk);
                const bool filter = readlane_i((int)nb_filter, nk) != 0;
                for (uint32_t base = beg; base < end; base += kChunk) {
                    const uint32_t m = end - base < (uint32_t)kChunk ? end - base : (uint32_t)kChunk;
                    // batches of 4 candidates per lane: loads first (index clamped to
                    // the chunk, so every load is in bounds), then branch-free tests
                    uint64_t acc = 0;
                    for (int i0 = 0; i0 < kChunk / L; i0 += 4) {
                        if ((uint32_t)(i0 * L) >= m) break;  // wave-uniform
                        float4 rc[4];
                        int4 cc[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint32_t k = q + (uint32_t)((i0 + u) * L);
                            const uint32_t kc = k < m ? k : m - 1;
                            rc[u] = srec[base + kc];
                            if constexpr (D == 3) cc[u] = scoord[base + kc];
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint32_t k = q + (uint32_t)((i0 + u) * L);
                            const float4 r = rc[u];
                            bool ok = in_group & (k < m);
                            if (filter) {
                                if constexpr (D == 2) {
                                    ok = ok & ((int64_t)__float_as_int(r.z) == n0) &
                                         ((int64_t)__float_as_int(r.w) == n1);
                                } else {
                                    ok = ok & ((int64_t)cc[u].x == n0) & ((int64_t)cc[u].y == n1) &
                                         ((int64_t)cc[u].z == n2);
                                }
                            }
                            const float d0 = delta_axis(pi[0], r.x, 0, P.g);
                            const float d1 = delta_axis(pi[1], r.y, 1, P.g);
                            float r2 = d0 * d0;
                            r2 += d1 * d1;
                            if constexpr (D == 3) {
                                const float d2 = delta_axis(pi[2], r.z, 2, P.g);
                                r2 += d2 * d2;
                            }
                            acc |= (ok & (r2 < P.g.eps2)) ? (1ull << (k & 63u)) : 0ull;
                        }
                    }
                    acc = group_or<L>(acc);
                    const uint32_t add = (uint32_t)__popcll(acc);
                    if (__ballot(cnt + add > CAP)) flush();
                    uint64_t mine = acc & my_residue;
                    while (mine) {
                        const uint32_t k = (uint32_t)__builtin_ctzll(mine);
                        mine &= mine - 1;
                        const uint32_t pos = cnt + (uint32_t)__popcll(acc & ((1ull << k) - 1ull));
                        lists.slot[pos][t] = base + k;
                    }
                    cnt += add;
                }
            }
        }
        flush();
        if (!active) continue;

        if (want_sg) {
            if (want_m) {  // apply_moment_correction normalize.rs:93-118
                float inv[D * D];
                safe_inverse<D>(mom, inv);
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
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
            for (int c = 0; c < CPL; ++c) {  // normalize_state_gradient normalize.rs:5-30
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
        // feature assembly forward.rs:100-133
        const uint32_t i = b * P.N + perm[s];
        float pp[3] = {0.0f, 0.0f, 0.0f};
        if (P.position_features) {
            const float4 p4 = io.pos[i];
            pp[0] = p4.x;
            pp[1] = p4.y;
            pp[2] = p4.z;
        }
        if constexpr (MODE == 0) {
            // padded layout [si SM][blur SM][grad SM*D][rest], feature-major; rest holds the
            // density gradient and/or position (runtime count) followed by zeros.
            const uint32_t T = P.T;
            float* f = sfeatures + row;
#pragma unroll
            for (int c = 0; c < CPL; ++c) f[(uint64_t)(c0 + c) * T] = si[c];
#pragma unroll
            for (int c = 0; c < CPL; ++c) f[(uint64_t)(SM + c0 + c) * T] = blur[c];
#pragma unroll
            for (int k = 0; k < CPL * D; ++k) f[(uint64_t)(2 * SM + c0 * D + k) * T] = want_sg ? grad[k] : 0.0f;
            if (q == 0) {
                float rest[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) rest[k] = 0.0f;
                int nr = 0;
                if (want_dg) {
#pragma unroll
                    for (int a = 0; a < D; ++a) rest[a] = dg[a];
                    nr = D;
                }
                if (P.position_features) {
#pragma unroll
                    for (int a = 0; a < D; ++a) {
                        if (nr == D) rest[D + a] = pp[a];
                        else rest[a] = pp[a];
                    }
                }
                constexpr uint32_t base_rest = 2 * SM + SM * D;
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    if (base_rest + r < P.FP) f[(uint64_t)(base_rest + r) * T] = rest[r];
            }
        } else {
            const uint32_t S = P.S;
            float* f = io.features + (uint64_t)i * P.F;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                if (c0 + c < S) {
                    f[c0 + c] = si[c];
                    f[S + c0 + c] = blur[c];
                    if (io.blurred) io.blurred[(uint64_t)i * S + c0 + c] = blur[c];
                    if (want_sg) {
#pragma unroll
                        for (int a = 0; a < D; ++a) {
                            f[2 * S + (c0 + c) * D + a] = grad[c * D + a];
                            if (io.state_gradient)
                                io.state_gradient[((uint64_t)i * S + c0 + c) * D + a] = grad[c * D + a];
                        }
                    }
                }
            if (q == 0) {
                uint32_t off = 2 * S + (want_sg ? S * D : 0);
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
                    for (int a = 0; a < D; ++a) f[off + a] = pp[a];
                }
            }
        }
    }
}

#if NPA_PART_MAIN
// Pads the model weights into the MLP kernel's layout, zeros everywhere else:
//   w1t [FP][HP]  w1 transposed, features at their padded positions, HP = H rounded up to 128
//   b1p [HP]
//   w2t [H][OP]   w2 transposed, OP = D + SS rounded up to a multiple of 4
//   b2p [OP]
__global__ __launch_bounds__(256) void k_pad_weights(StepParams P, int D, const float* __restrict__ w1,
                                                     const float* __restrict__ b1, const float* __restrict__ w2,
                                                     const float* __restrict__ b2, float* __restrict__ wpad) {
    const uint32_t S = P.S, SS = P.SS, F = P.F, H = P.H, FP = P.FP;
    const uint32_t HP = (H + 127) / 128 * 128;
    const uint32_t O = D + S, OP = (D + SS + 3) / 4 * 4;
    const uint64_t n1 = (uint64_t)FP * HP, n2 = (uint64_t)H * OP;
    const uint64_t total = n1 + HP + n2 + OP;
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (uint64_t)gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (k < n1) {
            const uint32_t q = (uint32_t)(k / HP), h = (uint32_t)(k - (uint64_t)q * HP);
            // padded feature position q -> real feature index
            int64_t fi = -1;
            if (q < SS) fi = q < S ? (int64_t)q : -1;
            else if (q < 2 * SS) fi = q - SS < S ? (int64_t)(S + q - SS) : -1;
            else if (q < 2 * SS + SS * D) {  // gradient features exist only with the state gradient
                const uint32_t g = q - 2 * SS;
                fi = P.state_grad && g < S * D ? (int64_t)(2 * S + g) : -1;
            } else {
                const uint32_t r = q - (2 * SS + SS * D);
                const uint32_t first = 2 * S + (P.state_grad ? S * D : 0);
                fi = first + r < F ? (int64_t)(first + r) : -1;
            }
            if (fi >= 0 && h < H) v = w1[(uint64_t)h * F + fi];
        } else if (k < n1 + HP) {
            const uint32_t h = (uint32_t)(k - n1);
            if (h < H) v = b1[h];
        } else if (k < n1 + HP + n2) {
            const uint64_t t = k - n1 - HP;
            const uint32_t h = (uint32_t)(t / OP), o = (uint32_t)(t - (uint64_t)h * OP);
            if (o < O) v = w2[(uint64_t)o * H + h];
        } else {
            const uint32_t o = (uint32_t)(k - n1 - HP - n2);
            if (o < O) v = b2[o];
        }
        wpad[k] = v;
    }
}

#endif  // NPA_PART_MAIN

// Update MLP + motion scaling + 3D gates + masked Euler for 64 sorted slots per 4-wave block.
// forward_update_from_features model.rs:900-940, forward_from_features_with_eps model.rs:867-898,
// gates model.rs:806-837, euler_step step.rs:4-55.
//   phase 1: lane = row; wave w computes hidden units [32w + 128p, 32w + 128p + 32) with the
//            weights of feature k as wave-uniform scalar loads; each hidden sum starts from its
//            bias and adds features k = 0..FM-1 in order (padded positions carry zero weights).
//   phase 2: lane = row; wave w owns outputs [OPW*w, OPW*w + OPW); each output sum starts from its
//            bias and adds hidden units h = 0..H-1 in order, reading them from LDS.
//   phase 3: wave 0 applies motion scaling, gates, mask and the Euler step for its 64 rows.
typedef float v4f __attribute__((ext_vector_type(4)));

// Phases 1 and 2 on the fp32 matrix cores (v_mfma_f32_16x16x4_f32: A 16x4, B 4x16, D 16x16;
// lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16]).
// Wave w serves rows 16w..16w+15 of the block's 64. Each accumulator starts from its bias; the
// matrix cores add the products in their own order, so the result differs from the reference's
// sequential sum in the last bits.
template <int FM, int OP>
__device__ __forceinline__ void mlp_mfma(const StepParams& P, const float* __restrict__ sfeatures, uint32_t row0,
                                         uint32_t nrows, uint32_t wave, uint32_t lane, const float* __restrict__ wpad,
                                         float* hid, float* ul) {
    const uint32_t H = P.H, T = P.T;
    const uint32_t HP = (H + 127) / 128 * 128;
    const float* w1t = wpad;
    const float* b1p = w1t + (uint64_t)FM * HP;
    const float* w2t = b1p + HP;
    const float* b2p = w2t + (uint64_t)H * OP;
    const uint32_t li = lane % 16, lk = lane / 16;
    const uint32_t rl = 16 * wave + li;          // block-local row this lane feeds as A
    const bool rvalid = row0 + rl < nrows;
    // layer 1: hidden = relu(b1 + F W1^T), 16 rows x HP hidden per wave, 16 columns per tile
    for (uint32_t hb = 0; hb < HP; hb += 128) {
        v4f acc[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float bias = b1p[hb + 16 * t + li];
            acc[t] = v4f{bias, bias, bias, bias};
        }
#pragma unroll 4
        for (int k0 = 0; k0 < FM; k0 += 4) {
            const uint32_t k = (uint32_t)k0 + lk;
            const float a = rvalid ? sfeatures[(uint64_t)k * T + row0 + rl] : 0.0f;
            const float* wk = w1t + (uint64_t)k * HP + hb + li;
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, wk[16 * t], acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                hid[(hb + 16 * t + li) * 64 + 16 * wave + 4 * lk + r] = fmaxf(acc[t][r], 0.0f);
    }
    __syncthreads();
    // layer 2: u = b2 + hidden W2^T, 16 rows x OP outputs per wave
    constexpr int OT = (OP + 15) / 16;
    v4f acc2[OT];
#pragma unroll
    for (int t = 0; t < OT; ++t) {
        const uint32_t col = 16 * t + li;
        const float bias = col < (uint32_t)OP ? b2p[col] : 0.0f;
        acc2[t] = v4f{bias, bias, bias, bias};
    }
    for (uint32_t k0 = 0; k0 < HP; k0 += 4) {
        const uint32_t k = k0 + lk;
        const float a = hid[k * 64 + rl];
#pragma unroll
        for (int t = 0; t < OT; ++t) {
            const uint32_t col = 16 * t + li;
            const float b = (k < H && col < (uint32_t)OP) ? w2t[(uint64_t)k * OP + col] : 0.0f;
            acc2[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc2[t], 0, 0, 0);
        }
    }
#pragma unroll
    for (int t = 0; t < OT; ++t) {
        const uint32_t col = 16 * t + li;
        if (col < (uint32_t)OP)
#pragma unroll
            for (int r = 0; r < 4; ++r) ul[(16 * wave + 4 * lk + r) * (OP + 1) + col] = acc2[t][r];
    }
}

template <int D, int SM, int FM, int ENG>
__global__ __launch_bounds__(256) void k_mlp_euler(StepParams P, const float* __restrict__ sfeatures,
                                                   const float* __restrict__ sstate,
                                                   const uint32_t* __restrict__ perm,
                                                   const uint32_t* __restrict__ act_rows,
                                                   const uint32_t* __restrict__ row_count,
                                                   const float* __restrict__ wpad, StepIO io) {
    constexpr int OP = (D + SM + 3) / 4 * 4;
    constexpr int OPW = OP / 4;
    extern __shared__ float lds[];
    const uint32_t H = P.H, T = P.T;
    const uint32_t HP = (H + 127) / 128 * 128;
    // LDS: hid [HP][64] (for HP = 128 the four waves' w1t slices [4][FM][32] share its region
    // before it is written); ul [64][OP + 1]; the VALU path's w2t copy [H][OP]
    float* hid = lds;
    const bool stage_w1 = HP == 128;  // one pass covers every hidden unit
    float* ul = lds + (stage_w1 && 4 * FM * 32 > HP * 64 ? (size_t)4 * FM * 32 : (size_t)HP * 64);
    const float* w1t = wpad;
    const float* b1p = w1t + (uint64_t)FM * HP;
    const float* w2t = b1p + HP;
    const float* b2p = w2t + (uint64_t)H * OP;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row0 = blockIdx.x * 64;
    const uint32_t nrows = *row_count;
    if (row0 >= nrows) return;  // whole block
    const uint32_t row = row0 + lane;
    const bool valid = row < nrows;
    const uint32_t s = act_rows[valid ? row : row0];  // sorted slot of this row's particle

    if constexpr (ENG == 1) {
        mlp_mfma<FM, OP>(P, sfeatures, row0, nrows, wave, lane, wpad, hid, ul);
    } else {
    float f[FM];
#pragma unroll
    for (int k = 0; k < FM; ++k) f[k] = valid ? sfeatures[(uint64_t)k * T + row] : 0.0f;

    // phase 1: hidden units. With one pass (HP = 128) each wave stages its 32-unit slice of w1t in
    // LDS (the region hid takes afterwards) and reads it back with broadcast loads, so no weight
    // load waits on L2; wider layers read w1t from memory.
    float* w2s = ul + 64 * (OP + 1);  // [H][OP]
    if (stage_w1) {
        float* w1s = lds + (size_t)wave * FM * 32;  // [FM][32] of this wave
        const uint32_t hb = wave * 32;
        for (uint32_t v = lane; v < (uint32_t)FM * 8; v += 64) {  // float4 v = (k, 4 units)
            const uint32_t k = v / 8, j4 = v % 8;
            reinterpret_cast<float4*>(w1s)[v] =
                *reinterpret_cast<const float4*>(w1t + (uint64_t)k * HP + hb + 4 * j4);
        }
        __syncthreads();
        float acc[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) acc[j] = b1p[hb + j];
#pragma unroll
        for (int k = 0; k < FM; ++k) {
            const float* wk = w1s + k * 32;
            const float fk = f[k];
#pragma unroll
            for (int j = 0; j < 32; ++j) acc[j] += wk[j] * fk;
        }
        __syncthreads();  // every wave has read its slice before hid overwrites the region
#pragma unroll
        for (int j = 0; j < 32; ++j) hid[(hb + j) * 64 + lane] = fmaxf(acc[j], 0.0f);
    } else {
        for (uint32_t hb = wave * 32; hb < HP; hb += 128) {
            float acc[32];
#pragma unroll
            for (int j = 0; j < 32; ++j) acc[j] = b1p[hb + j];
#pragma unroll
            for (int k = 0; k < FM; ++k) {
                const float* wk = w1t + (uint64_t)k * HP + hb;
                const float fk = f[k];
#pragma unroll
                for (int j = 0; j < 32; ++j) acc[j] += wk[j] * fk;
            }
#pragma unroll
            for (int j = 0; j < 32; ++j) hid[(hb + j) * 64 + lane] = fmaxf(acc[j], 0.0f);
        }
    }
    for (uint32_t v = threadIdx.x; v < H * OP / 4; v += blockDim.x)  // OP is a multiple of 4
        reinterpret_cast<float4*>(w2s)[v] = reinterpret_cast<const float4*>(w2t)[v];
    __syncthreads();

    // phase 2: outputs
    {
        const uint32_t ob = wave * OPW;
        float u[OPW];
#pragma unroll
        for (int o = 0; o < OPW; ++o) u[o] = b2p[ob + o];
        for (uint32_t h = 0; h < H; ++h) {
            const float hv = hid[h * 64 + lane];
            const float* wr = w2s + h * OP + ob;
#pragma unroll
            for (int o = 0; o < OPW; ++o) u[o] += wr[o] * hv;
        }
#pragma unroll
        for (int o = 0; o < OPW; ++o) ul[lane * (OP + 1) + ob + o] = u[o];
    }
    }  // ENG
    __syncthreads();
    if (wave != 0 || !valid) return;

    // phase 3: motion scaling, gates, mask, Euler
    const uint32_t S = P.S;
    float u[D + SM];
#pragma unroll
    for (int o = 0; o < D + SM; ++o) u[o] = ul[lane * (OP + 1) + o];
    const uint32_t b = s / P.N;
    const uint32_t li = perm[s];
    const uint32_t i = b * P.N + li;
    float norm = 0.0f;
#pragma unroll
    for (int a = 0; a < D; ++a) norm += u[a] * u[a];
    norm = sqrtf(norm);
    float dx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int a = 0; a < D; ++a) dx[a] = P.alpha * u[a] * P.motion_eps / (1.0f + norm);
    const float4 pos4 = io.pos[i];
    const float porig[4] = {pos4.x, pos4.y, pos4.z, pos4.w};
    float si[SM];
    {
        const float4* own = reinterpret_cast<const float4*>(sstate + (uint64_t)s * SM);
#pragma unroll
        for (int q = 0; q < SM / 4; ++q) {
            const float4 v = own[q];
            si[4 * q] = v.x;
            si[4 * q + 1] = v.y;
            si[4 * q + 2] = v.z;
            si[4 * q + 3] = v.w;
        }
    }
    float sg = 1.0f;
    if (P.gates3d) {
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
    const float m = io.mask ? io.mask[i] : hash_mask(li, b, P.N, P.update_prob, P.step_index, P.base_seed);
    float pn[4] = {porig[0], porig[1], porig[2], porig[3]};
    constexpr int MEM = D == 3 ? 4 : 2;
#pragma unroll
    for (int a = 0; a < MEM; ++a) pn[a] += P.dt * dx[a] * m;
    if (P.g.boundary == 0) {
#pragma unroll
        for (int a = 0; a < D; ++a) pn[a] = wrap_axis(pn[a], a, P.g);
    }
    io.out_pos[i] = make_float4(pn[0], pn[1], pn[2], pn[3]);
    float nxt[SM];
#pragma unroll
    for (int c = 0; c < SM; ++c) {
        float dsc = u[D + c];
        if (P.gates3d) dsc *= sg;
        float next = si[c] + P.dt * dsc * m;
        if (clamped_channel(D, S, (uint32_t)c)) next = clampf_(next, -8.0f, 24.0f);
        nxt[c] = next;
    }
    float* os = io.out_states + (uint64_t)i * S;
    if (S == SM) {  // 16-byte aligned rows (checked on the host)
        float4* o4 = reinterpret_cast<float4*>(os);
#pragma unroll
        for (int q = 0; q < SM / 4; ++q) o4[q] = make_float4(nxt[4 * q], nxt[4 * q + 1], nxt[4 * q + 2], nxt[4 * q + 3]);
    } else {
#pragma unroll
        for (int c = 0; c < SM; ++c)
            if ((uint32_t)c < S) os[c] = nxt[c];
    }
}

#if NPA_PART_MAIN
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
        for (int a = 0; a < g.dim; ++a) p[a] = wrap_axis(p[a], a, g);
    }
    out_pos[i] = make_float4(p[0], p[1], p[2], p[3]);
    for (uint32_t c = 0; c < S; ++c) {
        float next = states[i * S + c] + dt * ds[i * S + c] * m;
        if (clamped_channel(g.dim, S, c)) next = clampf_(next, -8.0f, 24.0f);
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

#endif  // NPA_PART_MAIN

// Candidates visited / pairs accepted by the neighbour walk (diagnostic, not on the step path):
// counters[0..1] over every particle (the density pass), counters[2..4] the targets of the step's
// hash update mask (P.update_prob, P.step_index), i.e. the second pass and the update MLP:
// [2] targets, [3] their candidates, [4] their pairs.
template <int D>
__global__ __launch_bounds__(256) void k_count_pairs(StepParams P, const float4* __restrict__ srec,
                                                     const int4* __restrict__ scoord,
                                                     const uint32_t* __restrict__ bo,
                                                     const uint32_t* __restrict__ perm,
                                                     const uint2* __restrict__ wl,
                                                     const uint32_t* __restrict__ wl_count,
                                                     unsigned long long* __restrict__ counters) {
    unsigned long long cand = 0, pairs = 0, targets = 0, tcand = 0, tpairs = 0;
    {
        NPA_WAVE_LOOP_BEGIN(wl, wl_count)
        const uint32_t b = s / P.N;
        float pi[3];
        int ci[3];
        load_rec<D>(srec, scoord, s, pi, ci);
        unsigned long long c = 0, pr = 0;
        constexpr int ZLO = D == 3 ? -1 : 0, ZHI = D == 3 ? 1 : 0;
        for (int dz = ZLO; dz <= ZHI; ++dz)
            for (int dy = -1; dy <= 1; ++dy)
                for (int dx = -1; dx <= 1; ++dx) {
                    uint32_t cell;
                    if (!cell_index((int64_t)ci[0] + dx, (int64_t)ci[1] + dy, (int64_t)ci[2] + dz, P.g, &cell))
                        continue;
                    const uint64_t bin = (uint64_t)b * P.g.cells + cell;
                    c += bo[bin + 1] - bo[bin];
                }
        walk_neighbors<D>(P.g, b, pi, ci, bo, srec, scoord, [&](uint32_t, const float*, float) { pr += 1; });
        cand += c;
        pairs += pr;
        if (hash_mask(perm[s], b, P.N, P.update_prob, P.step_index, P.base_seed) != 0.0f) {
            targets += 1;
            tcand += c;
            tpairs += pr;
        }
        NPA_WAVE_LOOP_END
    }
    atomicAdd(&counters[0], cand);
    atomicAdd(&counters[1], pairs);
    atomicAdd(&counters[2], targets);
    atomicAdd(&counters[3], tcand);
    atomicAdd(&counters[4], tpairs);
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
#if NPA_PART_MAIN
static StepParams with_directory(const StepParams& p, const Workspace& ws) {
    StepParams q = p;
    q.dir_n = ws.dir_n.as<uint32_t>();
    q.dir_e = ws.dir_e.as<int4>();
    return q;
}

hipError_t launch_density(const StepParams& p_in, Workspace& ws, float* density_out, int grid_blocks,
                          hipStream_t stream, Profiler* prof) {
    const StepParams p = with_directory(p_in, ws);
    // sparse grids (fewer than 4 particles per cell in 2D, fewer than 1 in 3D): a wave per cell run
    // would leave most of its lanes idle, so each target takes a group of lanes. Systems of at most
    // 64 targets per CU (C1, C4): a 16-lane row per target, since those
    // passes are set by their memory round trips (C1 9.3 -> 6.7 us, C4 32.0 -> 16.5 us against four
    // lanes per target); larger ones (C5: 38.0 against 53.4 us) keep four lanes, the fewer
    // instructions per candidate
    const bool rows = (uint64_t)p.T <= 64ull * (uint64_t)device_cu_count();
    const bool sparse = p.g.dim == 2 ? (uint64_t)p.B * p.g.cells * 4 > p.T : (uint64_t)p.B * p.g.cells > p.T;
    if (sparse && rows) {
        const uint32_t waves = (p.T + 3) / 4;
        auto k = p.g.dim == 2 ? k_density_rows<2> : k_density_rows<3>;
        return launch_timed(prof, NPA_KERNEL_DENSITY, k, dim3((waves + 3) / 4), dim3(256), 0, stream, p,
                            ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(),
                            ws.perm.as<uint32_t>(), ws.row_of.as<uint32_t>(), ws.svol.as<float4>(), density_out,
                            ws.nb_base.as<uint32_t>(), ws.nb_mask.as<uint64_t>(), ws.nb_count.as<uint32_t>());
    }
    if (p.g.dim == 2 && (uint64_t)p.B * p.g.cells * 4 > p.T) {  // four lanes per target, 16 per wave
        const uint32_t waves = (p.T + 15) / 16;
        return launch_timed(prof, NPA_KERNEL_DENSITY, k_density_lanes<2>, dim3((waves + 3) / 4), dim3(256), 0, stream,
                            p, ws.srec.as<float4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                            ws.row_of.as<uint32_t>(), ws.svol.as<float4>(), density_out, ws.nb_base.as<uint32_t>(),
                            ws.nb_mask.as<uint64_t>(), ws.nb_count.as<uint32_t>());
    }
    if (p.g.dim == 3 && (uint64_t)p.B * p.g.cells > p.T) {  // sparse 3D (more cells than particles)
        const uint32_t waves = (p.T + 15) / 16;
        return launch_timed(prof, NPA_KERNEL_DENSITY, k_density_lanes3, dim3((waves + 3) / 4), dim3(256), 0, stream,
                            p, ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(),
                            ws.perm.as<uint32_t>(), ws.row_of.as<uint32_t>(), ws.svol.as<float4>(), density_out,
                            ws.nb_base.as<uint32_t>(), ws.nb_mask.as<uint64_t>(), ws.nb_count.as<uint32_t>());
    }
    auto k = p.g.dim == 2 ? k_density_q<2> : k_density_q<3>;  // four waves per block, a wave per item
    return launch_timed(prof, NPA_KERNEL_DENSITY, k, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                        ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                        ws.row_of.as<uint32_t>(), ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(),
                        ws.svol.as<float4>(), density_out, ws.nb_base.as<uint32_t>(), ws.nb_mask.as<uint64_t>(),
                        ws.nb_count.as<uint32_t>());
}

#endif  // NPA_PART_MAIN

template <int D, int SM, int MODE, int FL>
static hipError_t launch_perceive_f(const StepParams& p, Workspace& ws, const StepIO& io, int blocks,
                                    hipStream_t stream, Profiler* prof) {
    return launch_timed(prof, NPA_KERNEL_PERCEIVE, k_perceive<D, SM, MODE, FL>, dim3(blocks), dim3(64), 0, stream, p, ws.srec.as<float4>(),
                       ws.scoord.as<int4>(), ws.sstate.as<float>(), ws.svol.as<float4>(),
                       ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(), ws.act_rows.as<uint32_t>(),
                       ws.wl_count.as<uint32_t>() + 1, ws.nb_base.as<uint32_t>(), ws.nb_mask.as<uint64_t>(),
                       ws.nb_count.as<uint32_t>(), ws.features.as<float>(), io);
}

// The rollout step's usual option sets run a specialised kernel; anything else reads the flags.
template <int D, int SM, int MODE>
static hipError_t launch_perceive_t(const StepParams& p, Workspace& ws, const StepIO& io, int blocks,
                                    hipStream_t stream, Profiler* prof) {
    if (MODE == 0 && p.state_grad && p.hybrid && !p.density_grad)
        return launch_perceive_f<D, SM, MODE, 5>(p, ws, io, blocks, stream, prof);
    if (MODE == 0 && p.state_grad && p.hybrid && p.density_grad)
        return launch_perceive_f<D, SM, MODE, 7>(p, ws, io, blocks, stream, prof);
    return launch_perceive_f<D, SM, MODE, -1>(p, ws, io, blocks, stream, prof);
}

template <int D, int MODE>
static hipError_t launch_perceive_d(const StepParams& p, Workspace& ws, const StepIO& io, int blocks,
                                    hipStream_t stream, Profiler* prof) {
    switch (p.SS) {
        case 4: return launch_perceive_t<D, 4, MODE>(p, ws, io, blocks, stream, prof);
        case 8: return launch_perceive_t<D, 8, MODE>(p, ws, io, blocks, stream, prof);
        case 16: return launch_perceive_t<D, 16, MODE>(p, ws, io, blocks, stream, prof);
        case 24: return launch_perceive_t<D, 24, MODE>(p, ws, io, blocks, stream, prof);
        default: return launch_perceive_t<D, 32, MODE>(p, ws, io, blocks, stream, prof);
    }
}

#if NPA_PART_MAIN
size_t valu_weight_floats(const StepParams& p) {
    const uint32_t D = (uint32_t)p.g.dim;
    const size_t HP = (p.H + 127) / 128 * 128;
    const size_t OP = (D + p.SS + 3) / 4 * 4;
    return ((size_t)p.FP * HP + HP + (size_t)p.H * OP + OP + 3) / 4 * 4;  // the fused layout stays 16-byte aligned
}

size_t padded_weight_floats(const StepParams& p) { return valu_weight_floats(p) + fused_weight_floats(p); }

bool fused_update_applies(const StepParams& p) {
    return p.SS == 16 && p.H <= 128 && (uint64_t)p.T * 64 < (1ull << 32);
}

hipError_t launch_pad_weights(const StepParams& p, const float* w1, const float* b1, const float* w2,
                              const float* b2, float* wpad, hipStream_t stream) {
    const size_t n = valu_weight_floats(p);
    const uint32_t blocks = (uint32_t)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(k_pad_weights, dim3(blocks), dim3(256), 0, stream, p, p.g.dim, w1, b1, w2, b2, wpad);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_pad_weights_fused(p, w1, b1, w2, b2, wpad + n, stream);
}

#endif  // NPA_PART_MAIN

template <int D, int SM, int FM, int ENG>
static hipError_t launch_mlp_e(const StepParams& p, Workspace& ws, const StepIO& io, hipStream_t stream,
                               Profiler* prof) {
    constexpr int OP = (D + SM + 3) / 4 * 4;
    const size_t HP = (p.H + 127) / 128 * 128;
    // hid [HP][64] (the VALU path first holds the four waves' w1t slices there), ul [64][OP+1],
    // then the VALU path's w2t copy [H][OP]
    const size_t hid_end = HP == 128 ? std::max<size_t>(HP * 64, 4 * (size_t)FM * 32) : HP * 64;
    const size_t lds = (hid_end + 64 * (OP + 1) + (ENG == 0 ? (size_t)p.H * OP : 0)) * 4;
    if (lds > 65536) {
        static LdsLimitFlags limit;
        const hipError_t e = raise_lds_limit((const void*)k_mlp_euler<D, SM, FM, ENG>, limit);
        if (e != hipSuccess) return e;
    }
    const uint32_t blocks = (p.T + 63) / 64;
    return launch_timed(prof, NPA_KERNEL_MLP, k_mlp_euler<D, SM, FM, ENG>, dim3(blocks), dim3(256), (uint32_t)lds,
                        stream, p, ws.features.as<float>(), ws.sstate.as<float>(), ws.perm.as<uint32_t>(),
                        ws.act_rows.as<uint32_t>(), ws.wl_count.as<uint32_t>() + 1, ws.wpad.as<float>(), io);
}

template <int D, int SM, int FM>
static hipError_t launch_mlp_t(const StepParams& p, Workspace& ws, const StepIO& io, hipStream_t stream,
                               Profiler* prof) {
    if (p.mlp_engine != NPA_MLP_VALU) return launch_mlp_e<D, SM, FM, 1>(p, ws, io, stream, prof);
    return launch_mlp_e<D, SM, FM, 0>(p, ws, io, stream, prof);
}

template <int D, int SM>
static hipError_t launch_mlp_sm(const StepParams& p, Workspace& ws, const StepIO& io, hipStream_t stream,
                                Profiler* prof) {
    constexpr int base = 2 * SM + SM * D;
    if (p.FP == (uint32_t)base) return launch_mlp_t<D, SM, base>(p, ws, io, stream, prof);
    if (p.FP == (uint32_t)base + 4) return launch_mlp_t<D, SM, base + 4>(p, ws, io, stream, prof);
    return launch_mlp_t<D, SM, base + 8>(p, ws, io, stream, prof);
}

template <int D>
static hipError_t launch_mlp_d(const StepParams& p, Workspace& ws, const StepIO& io, hipStream_t stream,
                               Profiler* prof) {
    switch (p.SS) {
        case 4: return launch_mlp_sm<D, 4>(p, ws, io, stream, prof);
        case 8: return launch_mlp_sm<D, 8>(p, ws, io, stream, prof);
        case 16: return launch_mlp_sm<D, 16>(p, ws, io, stream, prof);
        case 24: return launch_mlp_sm<D, 24>(p, ws, io, stream, prof);
        default: return launch_mlp_sm<D, 32>(p, ws, io, stream, prof);
    }
}

// Second pass, then (mode 0) the update MLP, for one dimension; the rollout step's usual shape
// (16-wide rows, H <= 128) runs both in the fused kernel, with either MLP engine.
template <int D>
static hipError_t launch_second_pass(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int blocks,
                                     hipStream_t stream, Profiler* prof) {
    if (mode == 0 && fused_update_applies(p)) {
        const float* wfused = ws.wpad.as<float>() + valu_weight_floats(p);
        return D == 2 ? launch_update_fused_2d(p, ws, io, wfused, stream, prof)
                      : launch_update_fused_3d(p, ws, io, wfused, stream, prof);
    }
    const hipError_t e = mode == 0 ? launch_perceive_d<D, 0>(p, ws, io, blocks, stream, prof)
                                   : launch_perceive_d<D, 1>(p, ws, io, blocks, stream, prof);
    if (e != hipSuccess || mode != 0) return e;
    return launch_mlp_d<D>(p, ws, io, stream, prof);
}

#if NPA_PART_DIM2
hipError_t launch_second_pass_2d(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int blocks,
                                 hipStream_t stream, Profiler* prof) {
    return launch_second_pass<2>(p, ws, io, mode, blocks, stream, prof);
}
#endif
#if NPA_PART_DIM3
hipError_t launch_second_pass_3d(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int blocks,
                                 hipStream_t stream, Profiler* prof) {
    return launch_second_pass<3>(p, ws, io, mode, blocks, stream, prof);
}
#endif

#if NPA_PART_MAIN
hipError_t launch_update(const StepParams& p_in, Workspace& ws, const StepIO& io, int mode, int grid_blocks,
                         hipStream_t stream, Profiler* prof) {
    const StepParams p = with_directory(p_in, ws);
    const int blocks = grid_blocks * 4;  // one wave per block
    return p.g.dim == 2 ? launch_second_pass_2d(p, ws, io, mode, blocks, stream, prof)
                        : launch_second_pass_3d(p, ws, io, mode, blocks, stream, prof);
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
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                           ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), counters);
    else
        hipLaunchKernelGGL(k_count_pairs<3>, dim3(grid_blocks), dim3(256), 0, stream, p, ws.srec.as<float4>(),
                           ws.scoord.as<int4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                           ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), counters);
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

#endif  // NPA_PART_MAIN

}  // namespace npa
