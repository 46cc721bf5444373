// npa_update.hip - the rollout step's second neighbour pass, update MLP and masked Euler step in
// one kernel, for sorted state rows of 16 channels (9 to 16 state channels) and H <= 128.
//
//   second pass   forward.rs:162-382 (blur_state, compute_state_gradient, moment_matrix,
//                 second_pass_particle), moment correction / scaling / log-norm normalize.rs:5-118,
//                 feature row forward.rs:100-133
//   update MLP    model.rs:900-940, motion scaling model.rs:867-898, 3D gates model.rs:806-837
//   Euler step    step.rs:4-55, written to the ping-pong output in original particle order
//
// Mapping. Sixteen lanes serve one target, lane c owning state channel c; a wave serves the four
// targets of one item (four consecutive compact rows); items are dealt round-robin over the grid's waves.
// The 16 waves of a block share the padded MLP weights in LDS.
//
// Per target, the accepted neighbours are appended to an LDS list in visit order (cells dz, dy, dx,
// slots ascending: the reference's for_each_neighbor order) from the density pass's per-chunk
// accept masks, or, for a target with more chunks than were recorded, by testing the candidates
// here. The list is consumed in rounds of 16 entries: lane c computes the pair scalars of entry c
// (poly6, volume, spiky gradient, moment terms) once; every lane then adds the round's 16 entries in
// list order to its own channel, reading the entry's scalars from lane e of its 16-lane row through
// DPP row_newbcast inside each multiply (the generic option set stages them in LDS instead) and the
// neighbour's channel from the sorted state rows. The per-target sums
// that are not per channel (moment matrix, density gradient) are summed by lane k for component k
// from a component-major copy of the round's terms. Padding entries (a short last round) use the
// target itself with zero weights. Every sum therefore adds the reference's terms in the reference's
// order, with the same roundings, and +0.0 terms that change nothing (each sum starts at +0.0).
//
// After the walk, lane l of the wave computes hidden units l and l + 64 of its four targets (bias
// first, then features in index order) and the hidden activations go to LDS; then lane c of a target
// sums output D + c (its state channel's update) and, for c < D, motion output c, hidden units in
// index order. The VALU engine rounds every product and sum as the reference does; the matrix-core
// engine (v_mfma_f32_4x4x1f32, same mapping) fuses each multiply-add and splits each sum into
// independent chains; the bf16 matrix-core engine (2D) runs layer 1 on v_mfma_f32_4x4x4bf16_1k with
// each feature split into three bf16 parts (hi + mid + lo = the feature exactly) and the weights
// rounded to bf16, so that for bf16-valued weights every product is exact and only the order of the
// fp32 sums differs. Lane 0 writes the position, every lane its state channel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "npa_internal.hpp"
#include "npa_neighbors.hpp"

#ifndef NPA_PART
#define NPA_PART -1
#endif
#define NPA_PART_MAIN (NPA_PART < 0 || NPA_PART == 0)
#define NPA_PART_DIM2 (NPA_PART < 0 || NPA_PART == 2)
#define NPA_PART_DIM3 (NPA_PART < 0 || NPA_PART == 3)

namespace npa {

constexpr int kFuseWaves = 16;          // waves per block (one block per CU)
constexpr uint32_t kFuseHidden = 128;   // hidden units held per target (H <= 128, zero padded)
constexpr uint32_t kFuseLdsBytes = 163840;

// Per-variant shapes. FL: option flags fixed at compile time (bit 0 state gradient, bit 1 density
// gradient, bit 2 moment correction, bit 3 periodic boundary; 5 = the rollout's usual set in a
// clamped domain, 13 the same in a periodic one) or -1 (read from the params). The clamped variant
// carries none of the periodic wrap's loop invariants (the fmod's divisor scaling, the extents),
// which keeps six more values out of scratch (C2 update 89 -> 87 us, 57 -> 47 MB per launch).
template <int D, int FL>
struct FuseShape {
    static constexpr int NMOM = D * (D + 1) / 2;            // moment matrix, upper triangle
    static constexpr bool COMMON = FL >= 0 && (FL & 7) == 5;
    static constexpr int SREC = COMMON ? 4 : 8;           // floats staged per entry
    static constexpr int NX = COMMON ? NMOM : NMOM + D;   // per-target sums over entries
    static constexpr int CAP = D == 2 ? (COMMON ? 256 : 160) : (COMMON ? 128 : 64);  // list entries
    static constexpr int OPAD = (D + 16 + 3) / 4 * 4;      // padded update outputs
    // Per wave, one block per target group g, one after the other: its list [CAP] u32, its entry
    // records [16][SREC] and its sums' terms [NX][XSTR] (so one address per lane reaches all three
    // through immediate offsets). Each part and each term row is padded by 4 floats, and the
    // blocks' stride keeps the four groups' broadcast reads of one offset in different LDS banks.
    // After the walk the same region holds the feature rows [4][FP + 4] and hidden activations
    // [4][132].
    static constexpr int LSTR = CAP + 4;
    static constexpr int SSTR = 16 * SREC + 4;
    static constexpr int XSTR = 20;
    static constexpr int XGSTR = NX * XSTR + 4;
    static constexpr int HSTR = 128 + 4;
    // a group's block: its three parts, plus 4 floats when their sum is a multiple of 16 floats
    // (then two groups' same offsets would share banks)
    static constexpr int GSTR = LSTR + SSTR + XGSTR + ((LSTR + SSTR + XGSTR) % 16 == 0 ? 4 : 0);
    static constexpr int WAVE_FLOATS = 4 * GSTR;
    static_assert(4 * (88 + 4 + HSTR) <= WAVE_FLOATS, "feature and hidden rows fit the wave's region");
};

// Floats of the fused MLP's padded weights: w1q [FP/4][128][4], b1 [128], w2q [32][OPAD][4], b2 [OPAD].
__host__ __device__ inline size_t fused_weight_floats(uint32_t FP, int dim) {
    const size_t opad = (size_t)(dim + 16 + 3) / 4 * 4;
    return (size_t)FP * kFuseHidden + kFuseHidden + kFuseHidden * opad + opad;
}

// Padded feature position q (16-wide rows) -> the model's feature index, or -1 for padding:
// [state 16][blur 16][gradient 16 x D][density gradient D?, position D?, zeros].
__device__ __forceinline__ int fused_feature_index(uint32_t q, const StepParams& P, int D) {
    const uint32_t S = P.S;
    if (q < 16) return q < S ? (int)q : -1;
    if (q < 32) return q - 16 < S ? (int)(S + q - 16) : -1;
    if (q < 32 + 16 * (uint32_t)D) {
        const uint32_t c = (q - 32) / D, a = (q - 32) % D;
        return P.state_grad && c < S ? (int)(2 * S + c * D + a) : -1;
    }
    const uint32_t r = q - (32 + 16 * D);
    const uint32_t nrest = (P.density_grad ? D : 0) + (P.position_features ? D : 0);
    return r < nrest ? (int)(2 * S + (P.state_grad ? S * D : 0) + r) : -1;
}

#if NPA_PART_MAIN
__global__ __launch_bounds__(256) void k_pad_weights_fused(StepParams P, int D, const float* __restrict__ w1,
                                                           const float* __restrict__ b1,
                                                           const float* __restrict__ w2,
                                                           const float* __restrict__ b2, float* __restrict__ wf) {
    const uint32_t H = P.H, F = P.F, FP = P.FP, O = D + P.S;
    const uint32_t HP = kFuseHidden, OPAD = (D + 16 + 3) / 4 * 4;
    const uint64_t n1 = (uint64_t)FP * HP, n2 = (uint64_t)HP * OPAD;
    const uint64_t total = n1 + HP + n2 + OPAD;
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < total; k += (uint64_t)gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (k < n1) {  // ((kb * HP + h) * 4 + i): feature 4 kb + i of hidden unit h
            const uint32_t i = (uint32_t)(k & 3), h = (uint32_t)((k >> 2) % HP), kb = (uint32_t)((k >> 2) / HP);
            const int fi = fused_feature_index(4 * kb + i, P, D);
            if (fi >= 0 && (uint32_t)fi < F && h < H) v = w1[(uint64_t)h * F + fi];
        } else if (k < n1 + HP) {
            const uint32_t h = (uint32_t)(k - n1);
            if (h < H) v = b1[h];
        } else if (k < n1 + HP + n2) {  // ((hb * OPAD + o) * 4 + i): hidden unit 4 hb + i of output o
            const uint64_t t = k - n1 - HP;
            const uint32_t i = (uint32_t)(t & 3), o = (uint32_t)((t >> 2) % OPAD), hb = (uint32_t)((t >> 2) / OPAD);
            const uint32_t h = 4 * hb + i;
            if (o < O && h < H) v = w2[(uint64_t)o * H + h];
        } else {
            const uint32_t o = (uint32_t)(k - n1 - HP - n2);
            if (o < O) v = b2[o];
        }
        wf[k] = v;
    }
}

hipError_t launch_pad_weights_fused(const StepParams& p, const float* w1, const float* b1, const float* w2,
                                    const float* b2, float* wf, hipStream_t stream) {
    const size_t n = fused_weight_floats(p.FP, p.g.dim);
    const uint32_t blocks = (uint32_t)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(k_pad_weights_fused, dim3(blocks), dim3(256), 0, stream, p, p.g.dim, w1, b1, w2, b2, wf);
    return hipGetLastError();
}

size_t fused_weight_floats(const StepParams& p) { return fused_weight_floats(p.FP, p.g.dim); }
#endif  // NPA_PART_MAIN

// Makes the wave's LDS writes visible to its other lanes before they read (a wave's LDS operations
// are performed in order; the barrier keeps the compiler from moving them across).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Value of `v` in lane (lane & ~15) + k: the same target's lane k.
// (DPP row_newbcast:k: no address register and no LDS round trip; k is a constant at every call
// once the loops are unrolled, and the switch folds to one move)
template <int K>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + K, 0xf, 0xf, false));
}
__device__ __forceinline__ float group_lane(float v, uint32_t lane, uint32_t k) {
    (void)lane;
    switch (k) {
        case 0: return row_bcast<0>(v);
        case 1: return row_bcast<1>(v);
        case 2: return row_bcast<2>(v);
        case 3: return row_bcast<3>(v);
        case 4: return row_bcast<4>(v);
        case 5: return row_bcast<5>(v);
        case 6: return row_bcast<6>(v);
        case 7: return row_bcast<7>(v);
        case 8: return row_bcast<8>(v);
        case 9: return row_bcast<9>(v);
        case 10: return row_bcast<10>(v);
        case 11: return row_bcast<11>(v);
        case 12: return row_bcast<12>(v);
        case 13: return row_bcast<13>(v);
        case 14: return row_bcast<14>(v);
        default: return row_bcast<15>(v);
    }
}

// Row-wise (16-lane) scans: row_shr:n reads lane i - n of the same row, 0 for the first n lanes.
template <int N>
__device__ __forceinline__ uint32_t row_shr(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + N, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t row_incl_sum(uint32_t v) {
    v += row_shr<1>(v);
    v += row_shr<2>(v);
    v += row_shr<4>(v);
    v += row_shr<8>(v);
    return v;
}
__device__ __forceinline__ uint32_t row_incl_max(uint32_t v) {
    v = max(v, row_shr<1>(v));
    v = max(v, row_shr<2>(v));
    v = max(v, row_shr<4>(v));
    v = max(v, row_shr<8>(v));
    return v;
}
// The row's last lane's value in every lane of the row (DPP row_newbcast:15).
__device__ __forceinline__ uint32_t row_last(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x150 + 15, 0xf, 0xf, false);
}

// One list entry of a round applied to this lane's channel: the entry's pair scalars live in lane E
// of the 16-lane row (the target's group), and each product reads them through DPP row_newbcast:E
// inside the multiply, so no LDS round trip and no extra instruction:
//   t0 = w[E] * x, t1 = vg0[E] * diff, t2 = vg1[E] * diff (, t3 = vg2[E] * diff).
// A DPP source must not have been written by the previous two VALU instructions (five after an
// EXEC write): the s_nop provides those wait states, since the compiler does not see inside asm.
template <int E, int D>
__device__ __forceinline__ void bcast_products(float w, float g0, float g1, float g2, float x, float diff, float& t0,
                                               float& t1, float& t2, float& t3) {
    if constexpr (D == 2) {
        asm volatile("s_nop %c8\n\t"
                     "v_mul_f32_dpp %0, %3, %6 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_mul_f32_dpp %1, %4, %7 row_newbcast:%c9 row_mask:0xf bank_mask:0xf\n\t"
                     "v_mul_f32_dpp %2, %5, %7 row_newbcast:%c9 row_mask:0xf bank_mask:0xf"
                     : "=&v"(t0), "=&v"(t1), "=&v"(t2)
                     : "v"(w), "v"(g0), "v"(g1), "v"(x), "v"(diff), "n"(E == 0 ? 4 : 1), "n"(E));
        t3 = 0.0f;
        (void)g2;
    } else {
        asm volatile("s_nop %c10\n\t"
                     "v_mul_f32_dpp %0, %4, %8 row_newbcast:%c11 row_mask:0xf bank_mask:0xf\n\t"
                     "v_mul_f32_dpp %1, %5, %9 row_newbcast:%c11 row_mask:0xf bank_mask:0xf\n\t"
                     "v_mul_f32_dpp %2, %6, %9 row_newbcast:%c11 row_mask:0xf bank_mask:0xf\n\t"
                     "v_mul_f32_dpp %3, %7, %9 row_newbcast:%c11 row_mask:0xf bank_mask:0xf"
                     : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
                     : "v"(w), "v"(g0), "v"(g1), "v"(g2), "v"(x), "v"(diff), "n"(E == 0 ? 4 : 1), "n"(E));
    }
}

template <typename F, int... E>
__device__ __forceinline__ void for_each_entry(F&& f, std::integer_sequence<int, E...>) {
    (f(std::integral_constant<int, E>{}), ...);
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));

// f32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN)
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ v4s as_v4s(uint2 v) { return __builtin_bit_cast(v4s, v); }

// Four features as three packed bf16 quads with hi + mid + lo == x exactly for finite x: each part
// takes the next eight significant bits of what the parts before it left (x - hi and its rest are
// exact in f32).
__device__ __forceinline__ void bf16x3_split(const float4& f, uint2& h, uint2& m, uint2& l) {
    const float x[4] = {f.x, f.y, f.z, f.w};
    uint32_t hb[4], mb[4], lb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hb[i] = bf16_rne(x[i]);
        const float r1 = x[i] - bf16_f32(hb[i]);
        mb[i] = bf16_rne(r1);
        lb[i] = bf16_rne(r1 - bf16_f32(mb[i]));
    }
    h = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
    m = make_uint2(mb[0] | (mb[1] << 16), mb[2] | (mb[3] << 16));
    l = make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16));
}

// ENG: 0 = VALU, the reference's roundings (bit-exact); 1 = the MLP on the fp32 matrix cores;
// 2 = layer 1 on the bf16 matrix cores (bf16x3 features, bf16 weights; 2D), layer 2 as ENG 1.
// NW: waves per block (kFuseWaves; small systems with the usual options take blocks of 4 so that
// their few items spread over every CU; a compile-time count keeps the item arithmetic in the
// scalar registers the kernel can spare).
template <int D, int FL, int ENG, int NW>
__global__ __launch_bounds__(1024) void k_update_fused(StepParams P, const float4* __restrict__ srec,
                                                       const int4* __restrict__ scoord,
                                                       const float* __restrict__ sstate,
                                                       const float4* __restrict__ svol,
                                                       const uint32_t* __restrict__ bo,
                                                       const uint32_t* __restrict__ perm,
                                                       const uint32_t* __restrict__ act_rows,
                                                       uint32_t* __restrict__ wlc,
                                                       const uint32_t* __restrict__ nb_base,
                                                       const uint64_t* __restrict__ nb_mask,
                                                       const uint32_t* __restrict__ nb_count,
                                                       const float* __restrict__ wfused, StepIO io) {
    using Sh = FuseShape<D, FL>;
    constexpr uint32_t CAP = Sh::CAP, SREC = Sh::SREC, NX = Sh::NX, NMOM = Sh::NMOM, OPAD = Sh::OPAD;
    constexpr uint32_t HP = kFuseHidden;
    constexpr uint32_t MAXC = max_chunks(D);
    extern __shared__ float lds[];
    const uint32_t FP = P.FP;
    const uint32_t wfloats = (uint32_t)fused_weight_floats(FP, D);

    // the block's copy of the padded weights (ENG 2: layer 1's as bf16 quads, w1b[FP/4][128], in the
    // first half of w1q's region)
    for (uint32_t v = threadIdx.x; v < wfloats / 4; v += blockDim.x) {
        const float4 x = reinterpret_cast<const float4*>(wfused)[v];
        if (ENG == 2 && v < FP * kFuseHidden / 4)
            reinterpret_cast<uint2*>(lds)[v] =
                make_uint2(bf16_rne(x.x) | (bf16_rne(x.y) << 16), bf16_rne(x.z) | (bf16_rne(x.w) << 16));
        else
            reinterpret_cast<float4*>(lds)[v] = x;
    }
    __syncthreads();
    const float* w1q = lds;
    const float* b1 = w1q + (size_t)FP * HP;
    const float* w2q = b1 + HP;
    const float* b2 = w2q + (size_t)HP * OPAD;

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, c = lane & 15;
    float* wl = lds + wfloats + (size_t)wave * Sh::WAVE_FLOATS;
    // this group's block: its list, its entry records, its sums' terms (one base per lane)
    float* gblk = wl + g * Sh::GSTR;
    uint32_t* mylist = reinterpret_cast<uint32_t*>(gblk);
    float* stage = gblk + Sh::LSTR;
    float* ext = gblk + Sh::LSTR + Sh::SSTR;
    float* hg = wl + 4 * (FP + 4) + g * Sh::HSTR;           // hidden activations (after the walk)

    const bool want_sg = FL >= 0 ? (FL & 1) != 0 : P.state_grad != 0;
    const bool want_dg = FL >= 0 ? (FL & 2) != 0 : P.density_grad != 0;
    const bool want_m = FL >= 0 ? (FL & 5) == 5 : (want_sg && P.hybrid);
    const bool periodic = FL >= 0 ? (FL & 8) != 0 : P.g.boundary == 0;
    // the pair's coordinate delta (neighbor_delta hashgrid.rs:165-181): a plain difference unless periodic
    auto delta = [&](float a, float bj, int ax) { return periodic ? delta_axis(a, bj, ax, P.g) : bj - a; };
    const bool branch_a = want_sg && want_dg;
    const uint32_t nrows = wlc[1];  // compact rows (update-mask targets)
    const uint32_t nitems = (nrows + 3) / 4;
    const uint32_t xcomp = c < NX ? c : 0u;  // the per-target sum this lane keeps

    // Items of four consecutive compact rows, in rounds of G * 16 consecutive items (neighbouring
    // rows share cells, so a CU's L1 and an XCD's L2 serve their neighbours once; a run of heavy
    // items, a dense region of the sorted order, is spread over many CUs). Blocks are dispatched to
    // the eight XCDs in turn: the blocks b with b % 8 == x share queue x, which hands out the x-th
    // eighth of every round (p-th position: round p / R, item round * G * 16 + x * R + p % R with
    // R = G / 8 * 16). Each wave's first position is dealt statically (block b's waves take
    // b / 8 * 16 + wave); later ones come from the queue's counter (zeroed with the work-list
    // counters by the hashgrid build) when an item is done, so the XCD's waves share its items to
    // the end, and a wave that the SIMD's oldest-first issue keeps waiting takes fewer of them.
    constexpr uint32_t nw = NW;
    const uint32_t nq = gridDim.x % 8 == 0 ? 8u : 1u;
    const uint32_t xq = blockIdx.x % nq;
    const uint32_t per_round = gridDim.x / nq * nw;
    auto item_at = [&](uint32_t p) { return (p / per_round) * (gridDim.x * nw) + xq * per_round + p % per_round; };
    uint32_t* queue = wlc + kQueueWord + xq * kQueueStride;
    auto take = [&]() {
        uint32_t p = 0;
        if (lane == 0) p = atomicAdd(queue, 1u);
        return per_round + (uint32_t)__builtin_amdgcn_readfirstlane((int)p);
    };
    auto slot_of = [&](uint32_t it) {
        const uint32_t r = it * 4 + g;
        return act_rows[r < nrows ? r : it * 4];
    };
    uint32_t item = item_at(blockIdx.x / nq * nw + wave);
    uint32_t s_next = item < nitems ? slot_of(item) : 0u;  // the item's compact-row slot
    while (item < nitems) {
        const uint32_t row = item * 4 + g;
        const bool active = row < nrows;
        const uint32_t s = s_next;
        // everything that depends only on the slot is issued together
        float pi[3];
        int ci[3];
        load_rec<D>(srec, scoord, s, pi, ci);
        const float si = sstate[(uint64_t)s * 16 + c];
        // the target's chunk records (contiguous per compact row); lane c holds chunk c (16 <= max_chunks)
        const uint32_t rrow = active ? row : item * 4;
        const uint32_t nct = active ? nb_count[rrow] : 0u;
        const uint32_t* rbase = nb_base + (uint64_t)rrow * MAXC;
        const uint64_t* rmask = nb_mask + (uint64_t)rrow * MAXC;
        const uint32_t base0 = rbase[c];
        const uint64_t mask0 = rmask[c];
        const uint32_t li = perm[s];

        const uint32_t b = s / P.N;
        const uint32_t i = b * P.N + li;
        // (in 3D the position is loaded after the walk: held across it, it would spill)
        float4 pos4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (D == 2) pos4 = io.pos[i];
        float blur = 0.0f, gr[3] = {0.0f, 0.0f, 0.0f}, xacc = 0.0f;
        uint32_t cnt = 0;  // entries in this target's list

        // ---- Phase B: the lists in rounds of 16 entries. sv[e] holds the neighbour channel of entry
        // e of the current round; right after it is used, the same entry of the next round is loaded
        // into it, so every load has about one round to arrive.
        auto load_sv = [&](uint32_t slot) {
            return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(sstate) + ((slot << 6) | (c << 2)));
        };
        auto process = [&]() {
            if (!__ballot(cnt > 0u)) return;
            const uint32_t padded = cnt == 0 ? 16u : (cnt + 15u) & ~15u;
            if (cnt + c < padded) mylist[cnt + c] = s;  // whole rounds; padding entries are the target
            const uint32_t nrg = padded / 16;           // a target with fewer rounds re-reads its last
            uint32_t nr = (uint32_t)__builtin_amdgcn_readlane((int)nrg, 0);
            nr = max(nr, (uint32_t)__builtin_amdgcn_readlane((int)nrg, 16));
            nr = max(nr, (uint32_t)__builtin_amdgcn_readlane((int)nrg, 32));
            nr = max(nr, (uint32_t)__builtin_amdgcn_readlane((int)nrg, 48));
            wave_sync();
            float sv[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = reinterpret_cast<const uint4*>(mylist)[q];
                sv[4 * q] = load_sv(v.x);
                sv[4 * q + 1] = load_sv(v.y);
                sv[4 * q + 2] = load_sv(v.z);
                sv[4 * q + 3] = load_sv(v.w);
            }
            uint32_t en = mylist[c];
            float4 rj = svol[en];
            // rounds in which this lane's entry 16 r + c is a list entry: r < lim
            const uint32_t lim = active && cnt > c ? (cnt - c + 15u) / 16u : 0u;
            for (uint32_t r = 0; r < nr; ++r) {
                const uint32_t rn = min(r + 1, nrg - 1);  // next round (always a valid entry; nrg >= 1)
                const uint32_t* lpn = mylist + 16 * rn;
                // this lane's entry: pair scalars, branch-free; a padding entry gets zero weights
                const bool has = r < lim;
                float d[3];
                d[0] = delta(pi[0], rj.x, 0);
                d[1] = delta(pi[1], rj.y, 1);
                d[2] = 0.0f;
                float r2 = d[0] * d[0];
                r2 += d[1] * d[1];
                if constexpr (D == 3) {
                    d[2] = delta(pi[2], rj.z, 2);
                    r2 += d[2] * d[2];
                }
                const float smooth = has ? poly6(r2, P.g) : 0.0f;
                const float vol = has ? rj.w : 0.0f;
                const bool gok = has && en != s && r2 > 0.0f;  // spiky_gradient_kernel kernels.rs:79-96
                const float rr = sqrtf(r2);
                const float tt = P.g.eps - rr;
                float vg[3] = {0.0f, 0.0f, 0.0f}, dgv[3] = {0.0f, 0.0f, 0.0f};
                if (want_dg) {
                    const float mag = 1.0f * P.g.k5 * 3.0f * (tt * tt) / rr;
#pragma unroll
                    for (int a = 0; a < D; ++a) dgv[a] = gok ? mag * d[a] : 0.0f;
                }
                if (want_sg) {
                    const float mag = rj.w * P.g.k5 * 3.0f * (tt * tt) / rr;
#pragma unroll
                    for (int a = 0; a < D; ++a) vg[a] = gok ? mag * d[a] : 0.0f;
                }
                const float w = smooth * vol;  // blur_state weight (density-grad-off branch)
                float* my = stage + c * SREC;
                if constexpr (SREC == 8) {  // (four floats per entry travel by DPP broadcast instead)
                    *reinterpret_cast<float4*>(my) = make_float4(branch_a ? smooth : w, vol, vg[0], vg[1]);
                    *reinterpret_cast<float4*>(my + 4) = make_float4(vg[2], 0.0f, 0.0f, 0.0f);
                }
                float* xe = ext + c;
                {
                    uint32_t k = 0;  // moment terms delta[ra] * grad[ca], upper triangle
#pragma unroll
                    for (int ra = 0; ra < D; ++ra)
#pragma unroll
                        for (int ca = ra; ca < D; ++ca) xe[Sh::XSTR * k++] = d[ra] * vg[ca];
                    if constexpr (NX > NMOM) {
#pragma unroll
                        for (int a = 0; a < D; ++a) xe[Sh::XSTR * (NMOM + a)] = dgv[a];
                    }
                }
                en = lpn[c];
                rj = svol[en];  // the next round's entry
                wave_sync();
                // the round's entries in list order
                if constexpr (SREC == 4) {
                    uint32_t nslot[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 nx = reinterpret_cast<const uint4*>(lpn)[q];
                        nslot[4 * q] = nx.x;
                        nslot[4 * q + 1] = nx.y;
                        nslot[4 * q + 2] = nx.z;
                        nslot[4 * q + 3] = nx.w;
                    }
                    for_each_entry(
                        [&](auto ic) {
                            constexpr int e = decltype(ic)::value;
                            const float x = sv[e];
                            const float diff = x - si;
                            float t0, t1, t2, t3;
                            bcast_products<e, D>(w, vg[0], vg[1], vg[2], x, diff, t0, t1, t2, t3);
                            blur += t0;  // blur_state forward.rs:174-180 (x * w)
                            gr[0] += t1;  // compute_state_gradient forward.rs:297-333 (diff * grad)
                            gr[1] += t2;
                            if constexpr (D == 3) gr[2] += t3;
                            sv[e] = load_sv(nslot[e]);
                        },
                        std::make_integer_sequence<int, 16>{});
                } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 nx = reinterpret_cast<const uint4*>(lpn)[q];
                    const uint32_t nslot[4] = {nx.x, nx.y, nx.z, nx.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int e = 4 * q + i;
                        const float* re = stage + e * SREC;
                        const float4 r0 = *reinterpret_cast<const float4*>(re);
                        const float x = sv[e];
                        {
                            if (branch_a) blur += x * r0.x * r0.y;  // second_pass_particle forward.rs:263-270
                            else blur += x * r0.x;
                            if (want_sg) {
                                const float diff = x - si;
                                gr[0] += diff * r0.z;
                                gr[1] += diff * r0.w;
                                if constexpr (D == 3) gr[2] += diff * re[4];
                            }
                        }
                        sv[e] = load_sv(nslot[i]);
                    }
                }
                }
                {
                    const float4* xp = reinterpret_cast<const float4*>(ext + xcomp * Sh::XSTR);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 x = xp[q];
                        xacc += x.x;
                        xacc += x.y;
                        xacc += x.z;
                        xacc += x.w;
                    }
                }
                wave_sync();
            }
        };

        // ---- Phase A: the accepted candidates of each chunk (<= 64 consecutive slots of a cell run,
        // in visit order), appended to the lists; rounds are consumed whenever a chunk would not fit.
        // tested chunks: coordinate groups of the wave's targets, then each group's neighbour cells
        uint64_t pending = 0, grp = 0, cells = 0;
        int l0 = 0, l1 = 0, l2 = 0;
        uint32_t lb = 0, nb_beg = 0, nb_end = 0, cbase = 0, cend = 0;
        bool nb_filter = false, nb_found = false, cfilter = false;
        int64_t n0 = 0, n1 = 0, n2 = 0;
        auto next_cell = [&]() -> bool {
            while (cells) {
                const int nk = __ffsll((unsigned long long)cells) - 1;  // ascending = visit order
                cells &= cells - 1;
                n0 = (int64_t)l0 + nk % 3 - 1;
                n1 = (int64_t)l1 + (nk / 3) % 3 - 1;
                n2 = D == 3 ? (int64_t)l2 + nk / 9 - 1 : 0;
                cbase = (uint32_t)readlane_i((int)nb_beg, nk);
                cend = (uint32_t)readlane_i((int)nb_end, nk);
                cfilter = readlane_i((int)nb_filter, nk) != 0;
                if (cbase < cend) return true;
            }
            return false;
        };
        auto next_group = [&]() -> bool {
            while (pending) {
                const int leader = __ffsll((unsigned long long)pending) - 1;
                l0 = readlane_i(ci[0], leader);
                l1 = readlane_i(ci[1], leader);
                l2 = D == 3 ? readlane_i(ci[2], leader) : 0;
                lb = (uint32_t)readlane_i((int)b, leader);
                const bool same = active && ci[0] == l0 && ci[1] == l1 && (D == 2 || ci[2] == l2) && b == lb;
                grp = __ballot(same) & pending;
                pending &= ~grp;
                neighbor_runs<D>(P, bo, lb, l0, l1, l2, lane, nb_beg, nb_end, nb_filter, nb_found);
                cells = __ballot(nb_found);
                if (next_cell()) return true;
            }
            return false;
        };
        const bool recorded = !__ballot(nct > MAXC);
        if (recorded) {
            // lane c appends chunk k0 + c of its target: the group's chunks in order, each at the
            // running count plus the entries of the chunks before it; when a target's list would
            // overflow, the chunks that fit are appended, the lists consumed, and the rest follow
            for (uint32_t k0 = 0; __ballot(k0 < nct); k0 += 16) {
                const bool valid = k0 + c < nct;
                uint32_t cbase0 = base0;
                uint64_t m = mask0;
                if (k0 > 0 && valid) {
                    cbase0 = rbase[k0 + c];
                    m = rmask[k0 + c];
                }
                if (!valid) m = 0ull;
                uint32_t left = (uint32_t)__popcll(m);
                for (;;) {
                    const uint32_t incl = row_incl_sum(left);
                    const uint32_t room = CAP - cnt;
                    const bool fits = left > 0 && incl <= room;
                    if (fits) {
                        uint32_t pos = cnt + incl - left;
                        while (m) {
                            const uint32_t bit = (uint32_t)__builtin_ctzll(m);
                            m &= m - 1;
                            mylist[pos++] = cbase0 + bit;
                        }
                        left = 0;
                    }
                    cnt += row_last(row_incl_max(incl <= room ? incl : 0u));  // the entries that fit
                    if (!__ballot(left > 0)) break;
                    process();
                    cnt = 0;
                }
            }
            process();
            cnt = 0;
        }
        bool more = false;
        if (!recorded) {
            pending = __ballot(active);
            more = next_group();
        }
        bool have = false;
        uint64_t acc = 0;
        uint32_t abase = 0;
        for (;;) {
            for (;;) {
                if (!have) {
                    if (!more) break;
                    {
                        const bool in_group = (grp >> lane) & 1ull;
                        const uint32_t m = cend - cbase < (uint32_t)kNbChunk ? cend - cbase : (uint32_t)kNbChunk;
                        acc = 0;
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint32_t k = c + 16u * u;
                            const uint32_t kc = k < m ? k : m - 1;
                            const float4 r = srec[cbase + kc];
                            bool ok = in_group & (k < m);
                            if (cfilter) {
                                if constexpr (D == 2) {
                                    ok = ok & ((int64_t)__float_as_int(r.z) == n0) & ((int64_t)__float_as_int(r.w) == n1);
                                } else {
                                    const int4 cc = scoord[cbase + kc];
                                    ok = ok & ((int64_t)cc.x == n0) & ((int64_t)cc.y == n1) & ((int64_t)cc.z == n2);
                                }
                            }
                            const float d0 = delta(pi[0], r.x, 0);
                            const float d1 = delta(pi[1], r.y, 1);
                            float r2 = d0 * d0;
                            r2 += d1 * d1;
                            if constexpr (D == 3) {
                                const float d2 = delta(pi[2], r.z, 2);
                                r2 += d2 * d2;
                            }
                            const uint64_t bal = __ballot(ok & (r2 < P.g.eps2));
                            acc |= ((bal >> (lane & 48u)) & 0xffffull) << (16 * u);
                        }
                        abase = cbase;
                        cbase += kNbChunk;
                        more = cbase < cend || next_cell() || next_group();
                    }
                    have = true;
                }
                if (__ballot(cnt + (uint32_t)__popcll(acc) > CAP)) break;
                // append: lane c takes bits c, c + 16, c + 32, c + 48 of the chunk's mask
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t bit = c + 16u * u;
                    if ((acc >> bit) & 1ull) {
                        const uint64_t below = (1ull << bit) - 1ull;
                        mylist[cnt + (uint32_t)__popcll(acc & below)] = abase + bit;
                    }
                }
                cnt += (uint32_t)__popcll(acc);
                have = false;
            }
            if (recorded) break;
            process();
            cnt = 0;
            if (!have && !more) break;
        }

        // ---- normalisation (normalize.rs:5-118) and the feature row
        float mom[D * D], dgs[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < D * D; ++k) mom[k] = 0.0f;
        {
            uint32_t k = 0;
#pragma unroll
            for (int ra = 0; ra < D; ++ra)
#pragma unroll
                for (int ca = ra; ca < D; ++ca) mom[ra * D + ca] = group_lane(xacc, lane, k++);
        }
        if constexpr (NX > NMOM) {
#pragma unroll
            for (int a = 0; a < D; ++a) dgs[a] = group_lane(xacc, lane, NMOM + a);
        }
        if (want_sg) {
            if (want_m) {  // apply_moment_correction normalize.rs:93-118
                float inv[D * D];
                safe_inverse<D>(mom, inv);
                float corrected[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int o = 0; o < D; ++o)
#pragma unroll
                    for (int k = 0; k < D; ++k) corrected[o] += gr[k] * inv[k * D + o];
#pragma unroll
                for (int o = 0; o < D; ++o) gr[o] = corrected[o];
            }
#pragma unroll
            for (int a = 0; a < D; ++a) gr[a] *= P.state_scale;  // normalize_state_gradient
            if (P.log_norm_grad) log_normalize<D>(gr);
        }
        if (want_dg) {  // normalize_density_gradient normalize.rs:32-58
#pragma unroll
            for (int a = 0; a < D; ++a) dgs[a] *= P.dgrad_scale;
            if (P.log_norm_dgrad) log_normalize<D>(dgs);
        }
        // feature row forward.rs:100-133: lane c of a target holds features c (state), 16 + c (blur)
        // and 32 + c D + a (gradient); the rest (density gradient, position, then zeros up to FP) is
        // the same in every lane of the target
        float rest[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) rest[k] = 0.0f;
        if constexpr (D == 3) pos4 = io.pos[i];
        {
            const float pp[3] = {pos4.x, pos4.y, pos4.z};
            int nrest = 0;
            if (want_dg) {
#pragma unroll
                for (int a = 0; a < D; ++a) rest[a] = dgs[a];
                nrest = D;
            }
            if (P.position_features) {
#pragma unroll
                for (int a = 0; a < D; ++a) {
                    if (nrest == D) rest[D + a] = pp[a];
                    else rest[a] = pp[a];
                }
            }
        }
        float gf[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) gf[a] = want_sg ? gr[a] : 0.0f;

        // ---- update MLP (model.rs:900-940), layer 1: lane l computes hidden units l and l + 64 of the
        // wave's four targets (each weight is read by one lane and used for four targets); feature k
        // of target t is read from the lane that holds it into a scalar register. Every sum starts
        // from its bias and adds the features in index order.
        constexpr uint32_t KB_FIXED = (32 + 16 * D) / 4;  // blocks of four state/blur/gradient features
        float* hw = wl + 4 * (FP + 4);  // hidden activations [target][HSTR]
        float us, um;
        {  // the four targets' feature rows [4][FP + 4]: lane l reads target l % 4's features
            float* fr = wl + g * (FP + 4);
            fr[c] = si;
            fr[16 + c] = blur;
#pragma unroll
            for (int a = 0; a < D; ++a) fr[32 + c * D + a] = gf[a];
            if (c == 0) {
#pragma unroll
                for (uint32_t k = 0; k < 8; ++k)
                    if (4 * KB_FIXED + k < FP) fr[4 * KB_FIXED + k] = rest[k];
            }
            wave_sync();
        }
        const float* myf = wl + (lane & 3u) * (FP + 4);
        if constexpr (ENG >= 1) {
            // Matrix-core engine (v_mfma_f32_4x4x1f32, 16 blocks of 4x4 with K = 1: lane l supplies
            // A[l / 4][l % 4] and B[l / 4][l % 4] and holds D[l / 4][r][l % 4] in accumulator r).
            // Layer 1: block b = hidden units 4b..4b+3, A = the four targets' feature k (lane l feeds
            // target l % 4), B = unit l's weight for feature k; lane l ends with unit l of targets
            // 0..3, the VALU mapping. The products are fused into the sums and the sums are split
            // into independent chains, so the result differs from the reference's in the last bits.
            const float* myf = wl + (lane & 3u) * (FP + 4);
            // Two independent accumulators per unit (even and odd feature pairs) keep four MFMA chains
            // in flight; they are added at the end, so this engine's sums are not in index order.
            const float bb0 = b1[lane], bb1 = b1[lane + 64];
            v4f a0 = {bb0, bb0, bb0, bb0}, a1 = {bb1, bb1, bb1, bb1};
            v4f c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = {0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (ENG == 2) {
                // v_mfma_f32_4x4x4bf16_1k, the same blocks with K = 4: lane l supplies features
                // 4kb..4kb+3 of target l % 4 (one bf16 part at a time) and unit l's bf16 weights for
                // them. The parts' rows [3][4 targets][FP / 4 quads] follow the hidden rows.
                const uint32_t nq = FP / 4;
                uint2* parts = reinterpret_cast<uint2*>(wl + 4 * (FP + 4) + 4 * Sh::HSTR);
                for (uint32_t v = lane; v < 4 * nq; v += 64) {
                    const uint32_t t = v / nq, qd = v - t * nq;
                    uint2 h, m, l;
                    bf16x3_split(*reinterpret_cast<const float4*>(wl + t * (FP + 4) + 4 * qd), h, m, l);
                    parts[t * nq + qd] = h;
                    parts[(4 + t) * nq + qd] = m;
                    parts[(8 + t) * nq + qd] = l;
                }
                wave_sync();
                const uint2* ph = parts + (lane & 3u) * nq;
                const uint2* pm = ph + 4 * nq;
                const uint2* pl = ph + 8 * nq;
                const uint2* w1b = reinterpret_cast<const uint2*>(w1q);
                for (uint32_t kb = 0; kb < nq; ++kb) {
                    const v4s wa = as_v4s(w1b[kb * HP + lane]), wb = as_v4s(w1b[kb * HP + lane + 64]);
                    const v4s xh = as_v4s(ph[kb]), xm = as_v4s(pm[kb]), xl = as_v4s(pl[kb]);
                    a0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xh, wa, a0, 0, 0, 0);
                    a1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xh, wb, a1, 0, 0, 0);
                    c0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xm, wa, c0, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xm, wb, c1, 0, 0, 0);
                    a0 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xl, wa, a0, 0, 0, 0);
                    a1 = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(xl, wb, a1, 0, 0, 0);
                }
            } else {
            auto mfma_block = [&](uint32_t kb) {
                const float4 f4 = *reinterpret_cast<const float4*>(myf + 4 * kb);
                const float4 w0 = *reinterpret_cast<const float4*>(w1q + ((size_t)kb * HP + lane) * 4);
                const float4 w1 = *reinterpret_cast<const float4*>(w1q + ((size_t)kb * HP + lane + 64) * 4);
                a0 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.x, w0.x, a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.x, w1.x, a1, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.y, w0.y, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.y, w1.y, c1, 0, 0, 0);
                a0 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.z, w0.z, a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.z, w1.z, a1, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.w, w0.w, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_4x4x1f32(f4.w, w1.w, c1, 0, 0, 0);
            };
#pragma unroll
            for (uint32_t kb = 0; kb < KB_FIXED; ++kb) mfma_block(kb);
            if (FP / 4 > KB_FIXED) mfma_block(KB_FIXED);
            if (FP / 4 > KB_FIXED + 1) mfma_block(KB_FIXED + 1);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                hw[t * Sh::HSTR + lane] = fmaxf(a0[t] + c0[t], 0.0f);
                hw[t * Sh::HSTR + lane + 64] = fmaxf(a1[t] + c1[t], 0.0f);
            }
            wave_sync();
            // Layer 2: block b = outputs 4b..4b+3 (blocks past OPAD / 4 compute copies of the last
            // output and are dropped), A = the four targets' hidden unit k, B = output l's weight
            // for unit k; lane l < OPAD ends with output l of targets 0..3.
            const uint32_t lo = lane < OPAD ? lane : OPAD - 1;
            const float* myh = hw + (lane & 3u) * Sh::HSTR;
            const float bo2 = b2[lo];
            v4f u2 = {bo2, bo2, bo2, bo2};  // four chains over the units 4 hb + i, summed at the end
            v4f u3 = {0.0f, 0.0f, 0.0f, 0.0f}, u4 = u3, u5 = u3;
#pragma unroll 8
            for (uint32_t hb = 0; hb < HP / 4; ++hb) {
                const float4 h4 = *reinterpret_cast<const float4*>(myh + 4 * hb);
                const float4 w4 = *reinterpret_cast<const float4*>(w2q + ((size_t)hb * OPAD + lo) * 4);
                u2 = __builtin_amdgcn_mfma_f32_4x4x1f32(h4.x, w4.x, u2, 0, 0, 0);
                u3 = __builtin_amdgcn_mfma_f32_4x4x1f32(h4.y, w4.y, u3, 0, 0, 0);
                u4 = __builtin_amdgcn_mfma_f32_4x4x1f32(h4.z, w4.z, u4, 0, 0, 0);
                u5 = __builtin_amdgcn_mfma_f32_4x4x1f32(h4.w, w4.w, u5, 0, 0, 0);
            }
            u2 = (u2 + u3) + (u4 + u5);
            // outputs [target][OPAD + 1] over the feature rows (read before the hidden rows were written)
            float* uo = wl;
            if (lane < OPAD) {
#pragma unroll
                for (int t = 0; t < 4; ++t) uo[t * (OPAD + 1) + lane] = u2[t];
            }
            wave_sync();
            us = uo[g * (OPAD + 1) + D + c];
            um = uo[g * (OPAD + 1) + (c < D ? c : 0u)];
        } else {
        // Layer 1, bit-exact: the products on the matrix cores, the sums on the vector ALUs. With a
        // -0.0 accumulator, v_mfma_f32_4x4x1f32 returns each product a * b rounded once - exactly
        // what v_mul_f32 returns, signed zeros and denormals included - laid out as the sums need
        // it (lane l: unit l of targets 0..3, as above); every sum then starts from its bias and
        // adds the products in feature order with separate roundings, as the reference does.
        float h0[4], h1[4];
        {
            const float bb0 = b1[lane], bb1 = b1[lane + 64];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                h0[t] = bb0;
                h1[t] = bb1;
            }
        }
        const v4f nzero = {-0.0f, -0.0f, -0.0f, -0.0f};
        auto prod_block = [&](uint32_t kb) {
            const float4 f4 = *reinterpret_cast<const float4*>(myf + 4 * kb);
            const float4 w0 = *reinterpret_cast<const float4*>(w1q + ((size_t)kb * HP + lane) * 4);
            const float4 w1 = *reinterpret_cast<const float4*>(w1q + ((size_t)kb * HP + lane + 64) * 4);
            const float fa[4] = {f4.x, f4.y, f4.z, f4.w};
            const float wa[4] = {w0.x, w0.y, w0.z, w0.w}, wb[4] = {w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4f p0 = __builtin_amdgcn_mfma_f32_4x4x1f32(fa[i], wa[i], nzero, 0, 0, 0);
                const v4f p1 = __builtin_amdgcn_mfma_f32_4x4x1f32(fa[i], wb[i], nzero, 0, 0, 0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    h0[t] += p0[t];
                    h1[t] += p1[t];
                }
            }
        };
#pragma unroll
        for (uint32_t kb = 0; kb < KB_FIXED; ++kb) prod_block(kb);
        if (FP / 4 > KB_FIXED) prod_block(KB_FIXED);
        if (FP / 4 > KB_FIXED + 1) prod_block(KB_FIXED + 1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            hw[t * Sh::HSTR + lane] = fmaxf(h0[t], 0.0f);
            hw[t * Sh::HSTR + lane + 64] = fmaxf(h1[t], 0.0f);
        }
        wave_sync();
        // outputs: state update D + c and motion output c (lanes c < D)
        us = b2[D + c];
        um = b2[c];
#pragma unroll 4
        for (uint32_t hb = 0; hb < HP / 4; ++hb) {
            const float4 h4 = *reinterpret_cast<const float4*>(hg + 4 * hb);
            const float4 ws4 = *reinterpret_cast<const float4*>(w2q + ((size_t)hb * OPAD + D + c) * 4);
            const float4 wm4 = *reinterpret_cast<const float4*>(w2q + ((size_t)hb * OPAD + c) * 4);
            us += ws4.x * h4.x;
            us += ws4.y * h4.y;
            us += ws4.z * h4.z;
            us += ws4.w * h4.w;
            um += wm4.x * h4.x;
            um += wm4.y * h4.y;
            um += wm4.z * h4.z;
            um += wm4.w * h4.w;
        }
        }
        wave_sync();  // the region is refilled by the next item

        // ---- motion scaling, gates, mask, Euler step (model.rs:806-898, step.rs:4-55)
        float u[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int a = 0; a < D; ++a) u[a] = group_lane(um, lane, a);
        float norm = 0.0f;
#pragma unroll
        for (int a = 0; a < D; ++a) norm += u[a] * u[a];
        norm = sqrtf(norm);
        float dx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int a = 0; a < D; ++a) dx[a] = P.alpha * u[a] * P.motion_eps / (1.0f + norm);
        float sgate = 1.0f;
        if (P.gates3d) {
            const float liveness = group_lane(si, lane, 3);
            const float sd = group_lane(si, lane, 7);
            sgate = clampf_((4.0f - liveness) * 2.0f, 0.0f, 1.0f);
            float mg;
            if (pos4.w >= 0.5f) {
                mg = 0.0f;
            } else {
                const float dgate = clampf_((fabsf(sd) - 0.01f) / 0.02f, 0.0f, 1.0f);
                mg = sgate * dgate;
            }
#pragma unroll
            for (int a = 0; a < D; ++a) dx[a] *= mg;
        }
        // every row is a target of the step's update mask: a mask array's value, or the hash mask's
        // 1.0 (the particles it zeroes get no row; the hashgrid build wrote them out unchanged)
        const float mk = io.mask ? io.mask[i] : 1.0f;
        if (active && c == 0) {
            float pn[4] = {pos4.x, pos4.y, pos4.z, pos4.w};
            constexpr int MEM = D == 3 ? 4 : 2;
#pragma unroll
            for (int a = 0; a < MEM; ++a) pn[a] += P.dt * dx[a] * mk;
            if (periodic) {
#pragma unroll
                for (int a = 0; a < D; ++a) pn[a] = wrap_axis(pn[a], a, P.g);
            }
            io.out_pos[i] = make_float4(pn[0], pn[1], pn[2], pn[3]);
        }
        float dsc = us;
        if (P.gates3d) dsc *= sgate;
        float next = si + P.dt * dsc * mk;
        if (clamped_channel(D, P.S, c)) next = clampf_(next, -8.0f, 24.0f);
        // (c passes through an empty asm so that out_states + c is formed here, per item, rather
        // than hoisted into a 64-bit register pair held across the whole loop)
        uint32_t cs = c;
        asm volatile("" : "+v"(cs));
        if (active && c < P.S) io.out_states[(uint64_t)i * P.S + cs] = next;
        item = item_at(take());
        if (item < nitems) s_next = slot_of(item);
    }
}

template <int D, int FL, int ENG, int NW>
static hipError_t launch_fused_t(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                 hipStream_t stream, Profiler* prof) {
    using Sh = FuseShape<D, FL>;
    // one block per CU at most; never more waves than items of four targets
    const uint64_t max_items = ((uint64_t)p.T + 3) / 4;
    const uint64_t cus = (uint64_t)device_cu_count();
    const size_t lds = (fused_weight_floats(p.FP, D) + (size_t)NW * Sh::WAVE_FLOATS) * 4;
    if (lds > kFuseLdsBytes) return hipErrorInvalidValue;
    static LdsLimitFlags limit;
    const hipError_t e = raise_lds_limit((const void*)k_update_fused<D, FL, ENG, NW>, limit);
    if (e != hipSuccess) return e;
    const uint32_t blocks = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(cus, (max_items + NW - 1) / NW));
    uint32_t* wl = ws.wl_count.as<uint32_t>();
    return launch_timed(prof, NPA_KERNEL_UPDATE, k_update_fused<D, FL, ENG, NW>, dim3(blocks), dim3(64 * NW),
                        (uint32_t)lds, stream, p, ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(),
                        ws.svol.as<float4>(), ws.bin_offsets.as<uint32_t>(), ws.perm.as<uint32_t>(),
                        ws.act_rows.as<uint32_t>(), wl, ws.nb_base.as<uint32_t>(),
                        ws.nb_mask.as<uint64_t>(), ws.nb_count.as<uint32_t>(), wfused, io);
}

template <int D>
static hipError_t launch_fused_d(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                 hipStream_t stream, Profiler* prof) {
    // the usual option set (flags 5), clamped or periodic (flag 8), or every option read at run time
    const bool common = p.state_grad && p.hybrid && !p.density_grad;
    const bool per = p.g.boundary == 0;
    constexpr int W = kFuseWaves;
    if constexpr (D == 2) {  // the bf16 engine (2D; its bf16 feature parts must fit the wave's region)
        constexpr uint32_t room = (uint32_t)std::min(FuseShape<2, 5>::WAVE_FLOATS, FuseShape<2, 13>::WAVE_FLOATS);
        if (p.mlp_engine == NPA_MLP_MFMA_BF16 && 10 * p.FP + 4 * (16 + FuseShape<2, 5>::HSTR) <= room &&
            10 * p.FP + 4 * (16 + FuseShape<2, -1>::HSTR) <= (uint32_t)FuseShape<2, -1>::WAVE_FLOATS)
            return !common ? launch_fused_t<D, -1, 2, W>(p, ws, io, wfused, stream, prof)
                   : per   ? launch_fused_t<D, 13, 2, W>(p, ws, io, wfused, stream, prof)
                           : launch_fused_t<D, 5, 2, W>(p, ws, io, wfused, stream, prof);
    }
    if (p.mlp_engine != NPA_MLP_VALU)
        return !common ? launch_fused_t<D, -1, 1, W>(p, ws, io, wfused, stream, prof)
               : per   ? launch_fused_t<D, 13, 1, W>(p, ws, io, wfused, stream, prof)
                       : launch_fused_t<D, 5, 1, W>(p, ws, io, wfused, stream, prof);
    // a system with at most four items per CU (C1: 4,096 particles): blocks of four waves, so that
    // its items spread over every CU instead of queueing on a few
    const bool small = ((uint64_t)p.T + 3) / 4 <= 4ull * (uint64_t)device_cu_count();
    if (common && small)
        return per ? launch_fused_t<D, 13, 0, 4>(p, ws, io, wfused, stream, prof)
                   : launch_fused_t<D, 5, 0, 4>(p, ws, io, wfused, stream, prof);
    return !common ? launch_fused_t<D, -1, 0, W>(p, ws, io, wfused, stream, prof)
           : per   ? launch_fused_t<D, 13, 0, W>(p, ws, io, wfused, stream, prof)
                   : launch_fused_t<D, 5, 0, W>(p, ws, io, wfused, stream, prof);
}

#if NPA_PART_DIM2
hipError_t launch_update_fused_2d(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                  hipStream_t stream, Profiler* prof) {
    return launch_fused_d<2>(p, ws, io, wfused, stream, prof);
}
#endif
#if NPA_PART_DIM3
hipError_t launch_update_fused_3d(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                  hipStream_t stream, Profiler* prof) {
    return launch_fused_d<3>(p, ws, io, wfused, stream, prof);
}
#endif

}  // namespace npa
