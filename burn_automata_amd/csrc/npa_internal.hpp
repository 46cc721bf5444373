// npa_internal.hpp - host-side interfaces between the library's translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include <string>
#include <vector>

#include "../../include/npa_abi.h"
#include "npa_device.hpp"

namespace npa {

// Grow-only device allocation, or a view into memory the library does not allocate (view(); never
// freed).
struct DevBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool owned = true;
    hipError_t reserve(size_t want);
    void release();
    void view(void* p, size_t b);
    template <class T>
    T* as() const { return static_cast<T*>(ptr); }
};

// Per-context profiling: HIP events bracket launches of selected kernels.
struct Profiler {
    bool enabled = false;
    uint32_t mask = 0;  // bit k selects kernel id k
    struct Pair { hipEvent_t a, b; int kernel; };
    std::vector<Pair> pending;
    std::vector<hipEvent_t> pool;
    double total_ms[NPA_KERNEL_COUNT] = {0};
    uint64_t launches[NPA_KERNEL_COUNT] = {0};
    hipEvent_t get();
    bool selects(int kernel) const { return enabled && ((mask >> kernel) & 1u); }
    // Start/stop events for one launch of `kernel`, queued for collect(); false when unavailable.
    bool pick(int kernel, hipEvent_t* a, hipEvent_t* b);
    void begin(int kernel, hipStream_t s, hipEvent_t* ev);
    void end(int kernel, hipStream_t s, hipEvent_t ev);
    hipError_t collect();  // synchronizes pending events into the totals
    void reset();
    ~Profiler();
};

// Launches `kernel`; when the profiler selects `kernel_id`, through hipExtLaunchKernelGGL with
// start/stop events that the dispatch itself timestamps, so the recorded time is the kernel's
// execution alone (no queue gaps or launch overhead).
template <class F, class... Args>
inline hipError_t launch_timed(Profiler* prof, int kernel_id, F kernel, dim3 grid, dim3 block, uint32_t shmem,
                               hipStream_t stream, Args... args) {
    hipEvent_t a = nullptr, b = nullptr;
    if (prof && prof->selects(kernel_id) && prof->pick(kernel_id, &a, &b))
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, a, b, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
    return hipGetLastError();
}

// Brackets a multi-kernel sequence with events recorded on the stream.
struct ProfScope {
    Profiler* p;
    int kernel;
    hipStream_t s;
    hipEvent_t ev = nullptr;
    ProfScope(Profiler* p_, int k, hipStream_t s_) : p(p_), kernel(k), s(s_) {
        if (p && p->enabled && ((p->mask >> kernel) & 1u)) p->begin(kernel, s, &ev);
    }
    ~ProfScope() {
        if (p && p->enabled && ev) p->end(kernel, s, ev);
    }
};

// How the hashgrid build splits the particles of one system into tiles.
struct HashgridPlan {
    uint32_t cells = 0;          // C
    uint32_t key_bits = 0;       // ceil(log2(C))
    uint32_t waves = 0;          // waves per tile (block)
    uint32_t rounds = 0;         // R: 64-particle rounds per wave
    uint32_t tile = 0;           // particles per tile = waves * rounds * 64
    uint32_t tiles_per_sys = 0;
    uint32_t lds_bytes = 0;      // waves * C * 2
    uint64_t table_entries = 0;  // B * tiles_per_sys * C
    uint64_t worklist_cap = 0;   // upper bound of wave work items
    uint32_t tpi = 64;           // targets (slots) per work item
};

// Device workspace of one hashgrid + perception pass.
// Bins are split by true cell for the neighbour passes: a bin holding up to kDirGroups distinct
// cells gets one contiguous run of slots per cell (ascending particle index inside each run) and a
// directory entry {cx, cy, cz, first slot} per run; dir_n[bin] = number of runs, or
// kDirGroups + 1 when the bin holds more cells and keeps the reference order.
constexpr uint32_t kDirGroups = 8;
constexpr uint32_t kListedWord = 32;  // wl_count word of the thin split's listed-bin count
constexpr uint32_t kQueueWord = 64;    // wl_count word of the fused update's first item queue
constexpr uint32_t kQueueStride = 32;  // words between queues (one 128-byte line each; eight queues)
constexpr uint32_t kWlWords = 512;     // wl_count words, all zeroed by the hashgrid build

struct Workspace {
    // flags: u32 [0] the current build's coordinate overflow (set by k_hash_rank, moved by
    // k_scatter), [1] overflows not yet reported (read and cleared by the synchronising calls)
    DevBuf keys, ranks, table, totals, bin_offsets, perm, inv, flags, wl_count, worklist;
    DevBuf srec, scoord, sstate, counters, features, wpad;
    // svol: per sorted slot float4 {x, y, z, 1/rho (recip_finite)}, written by the density pass:
    // the second pass gathers a neighbour's position and volume with one load
    DevBuf svol;
    DevBuf tmpidx, dir_n, dir_e;
    // one-pass offsets scan: per (system, 256-key block) the block's published key total
    // (bit 63 = published; zeroed by k_hash_rank at the start of every build)
    DevBuf scan_status;
    // sparse grids: the bins too large for the one-lane split (count in wl_count[kListedWord]); the
    // folded build's per-key row counters
    DevBuf bin_list;
    // the folded build: per rank tile, the cell coordinate span (min x, y, z, max x, y, z, 2 spare)
    DevBuf tile_span;
    // the binned build (one system): per bin a 64-bit counter (particles | update-mask targets << 32)
    // and after the C counters eight span words; all zero between builds (zeroed when allocated,
    // reset by the build's scan). bin_urow: per particle its target index within its bin (~0u for
    // a particle outside the mask).
    DevBuf bin_count, bin_urow;
    // Targets of the second pass and the update: particles whose update mask is not 0 (the others
    // are written to the output by the update-mask kernel). act_rows: compact row -> slot.
    // Counts (u32 words of wl_count, kWlWords): [0] density items, [1] compact rows (one 64-bit
    // word, so one atomic reserves both), [kListedWord] listed bins (another cache line, so its
    // atomics do not queue behind the reservations), [kQueueWord + x * kQueueStride] the fused
    // update's item queue of XCD x.
    DevBuf act_rows;
    // row_of: slot -> compact row of an update-mask target, or ~0u (written by the split).
    // Accepted neighbours recorded by the density pass for the targets, per neighbour chunk (<= 64
    // consecutive slots of a cell run, in visit order): the chunk's first slot (nb_base) and its
    // 64-bit accept mask (nb_mask) at [row * max_chunks(dim) + chunk] for the first max_chunks(dim)
    // chunks, and the chunk count at nb_count[row] (the second pass tests the candidates itself
    // when it exceeds the cap). A target's records are contiguous, so the second pass reads them
    // coalesced.
    DevBuf row_of, nb_base, nb_mask, nb_count;
    hipError_t reserve(const HashgridPlan& plan, uint64_t total, uint32_t batch, uint32_t state_dims,
                       int dim, uint32_t feature_dims = 0);
    // The same buffers (with wpad_bytes for the padded weights) as views into [base, base +
    // capacity): the flags first (kCarveFlagBytes), then every buffer on a 256-byte boundary. Returns
    // the bytes the layout needs; the views are set only when it fits (and base is not null).
    uint64_t carve(const HashgridPlan& plan, uint64_t total, uint32_t batch, uint32_t state_dims, int dim,
                   uint32_t feature_dims, uint64_t wpad_bytes, void* base, uint64_t capacity);
    void release();
};
constexpr uint64_t kCarveFlagBytes = 256;

// Chunk records kept per target by the density pass (a 2D target visits 9 cells, a 3D one 27; a
// cell run of more than 64 particles spans several chunks).
__host__ __device__ constexpr uint32_t max_chunks(int dim) { return dim == 3 ? 48u : 24u; }

// tpi: targets per wave work item emitted for the neighbour passes (the density pass serves one
// with four lanes per target).
bool make_plan(const npa_grid_cfg& cfg, uint32_t batch, uint32_t particle_count, HashgridPlan* plan,
               std::string* err, uint32_t tpi = 16);
GridParams make_grid_params(const npa_grid_cfg& cfg);
float host_powi(float x, int n);

// The particles a step's second pass and update MLP process: those whose update mask is not 0.
// The split kernel gives them consecutive compact rows (act_rows, count in wl_count[1]) and writes
// every other particle to the step's output with the Euler step's wrap / clamp only
// (hold_particle). mask_mode: 0 every particle (no copies), 1 the device hash mask, 2 a mask array.
struct SplitTargets {
    int mask_mode = 0;
    const float* mask = nullptr;
    float update_prob = 1.0f;
    uint32_t step_index = 0, base_seed = 0;
    const float4* pos = nullptr;
    const float* states = nullptr;
    float4* out_pos = nullptr;
    float* out_states = nullptr;
};

// Builds the stable hashgrid; when `payload` is set also the sorted particle records (positions
// + cell coords), sorted state rows, the density work list and the second pass's targets
// (`targets`, or every particle when null).
hipError_t launch_hashgrid(const HashgridPlan& plan, const GridParams& g, const float4* pos,
                           const float* states, uint32_t state_dims, uint32_t batch,
                           uint32_t particle_count, Workspace& ws, bool payload,
                           hipStream_t stream, Profiler* prof, const SplitTargets* targets = nullptr);
// the sorted state rows are written with stride state_stride_for(state_dims), zero padded

// Stable counting sort of a device-resident number (<= cap) of items by key in [0, C):
// out_vals[offsets[key] + rank] = vals[i] (or i when vals is null), offsets[C+1].
bool make_key_sort_plan(uint32_t cap, uint32_t C, HashgridPlan* plan);
hipError_t launch_key_sort(const HashgridPlan& plan, const uint32_t* keys, const uint32_t* vals,
                           const uint32_t* d_count, uint32_t cap, uint32_t* ranks, uint32_t* table,
                           uint32_t* totals, uint32_t* offsets, uint32_t* out_vals, uint32_t* flags,
                           hipStream_t stream);

// Row width of the sorted state copy: S rounded up to the kernels' template width, zero padded,
// so the neighbour loops run over a compile-time channel count without bounds guards.
__host__ __device__ inline uint32_t state_stride_for(uint32_t S) {
    return S <= 4 ? 4 : S <= 8 ? 8 : S <= 16 ? 16 : S <= 24 ? 24 : 32;
}
// Lanes per target in the neighbour passes (each lane owns SS / L state channels) and the
// targets per wave work item, 64 / L.
__host__ __device__ inline uint32_t lanes_per_target(uint32_t SS) { return SS >= 16 ? 4u : SS / 4; }
__host__ __device__ inline uint32_t targets_per_item(uint32_t SS) { return 64u / lanes_per_target(SS); }
// Copies a state row (every load issued before the stores); in 3D the opacity-logit channels are
// clamped on the way.
template <int NQ>
__device__ __forceinline__ void hold_state_row(float* __restrict__ dst, const float* __restrict__ src, int dim) {
    float4 v[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) v[q] = reinterpret_cast<const float4*>(src)[q];
    if (dim == 3) {
        v[0].w = clampf_(v[0].w, -8.0f, 24.0f);                               // channel 3
        if constexpr (NQ > 2) v[2].x = clampf_(v[2].x, -8.0f, 24.0f);          // channel 8 (S > 8)
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) reinterpret_cast<float4*>(dst)[q] = v[q];
}

// A particle whose update mask is 0. The CPU euler_step (step.rs:4-55) adds dt * d * 0 to each
// value, which is +-0 for a finite update and leaves every value but -0.0 unchanged, and then still
// applies the periodic wrap and the 3D opacity-logit clamp; those two are applied here, so the
// result equals the CPU path's without evaluating the update. (The reference's GPU update_particle,
// gpu_step.wgsl:3664-3682, copies such a particle without the wrap and the clamp.)
__device__ __forceinline__ void hold_particle(uint64_t i, uint32_t S, const GridParams& g,
                                              const float4* __restrict__ pos, const float* __restrict__ states,
                                              float4* __restrict__ out_pos, float* __restrict__ out_states) {
    float4 p = pos[i];
    if (g.boundary == 0) {
        p.x = wrap_axis(p.x, 0, g);
        p.y = wrap_axis(p.y, 1, g);
        if (g.dim == 3) p.z = wrap_axis(p.z, 2, g);
    }
    out_pos[i] = p;
    const float* src = states + i * S;
    float* dst = out_states + i * S;
    if (S == state_stride_for(S)) {  // 16-byte aligned rows (checked on the host)
        switch (S) {
            case 4: hold_state_row<1>(dst, src, g.dim); return;
            case 8: hold_state_row<2>(dst, src, g.dim); return;
            case 16: hold_state_row<4>(dst, src, g.dim); return;
            case 24: hold_state_row<6>(dst, src, g.dim); return;
            default: hold_state_row<8>(dst, src, g.dim); return;
        }
    }
    for (uint32_t c = 0; c < S; ++c) {
        const float v = src[c];
        dst[c] = clamped_channel(g.dim, S, c) ? clampf_(v, -8.0f, 24.0f) : v;
    }
}

// hold_particle for a particle whose position and state row (NQ float4s, 16-byte aligned rows) are
// already in registers.
template <int NQ>
__device__ __forceinline__ void hold_loaded(uint64_t i, float4 p, const float4 (&row)[NQ], const GridParams& g,
                                            float4* __restrict__ out_pos, float* __restrict__ out_states) {
    if (g.boundary == 0) {
        p.x = wrap_axis(p.x, 0, g);
        p.y = wrap_axis(p.y, 1, g);
        if (g.dim == 3) p.z = wrap_axis(p.z, 2, g);
    }
    out_pos[i] = p;
    float4 v[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) v[q] = row[q];
    if (g.dim == 3) {
        v[0].w = clampf_(v[0].w, -8.0f, 24.0f);                               // channel 3
        if constexpr (NQ > 2) v[2].x = clampf_(v[2].x, -8.0f, 24.0f);          // channel 8 (S > 8)
    }
    float4* o4 = reinterpret_cast<float4*>(out_states + i * (4 * NQ));
#pragma unroll
    for (int q = 0; q < NQ; ++q) o4[q] = v[q];
}

// Padded feature row used between the perception and MLP kernels:
// [state SS][blur SS][grad SS*d][density-grad d?, position d?, zero padded to a multiple of 4].
__host__ __device__ inline uint32_t padded_features(uint32_t SS, uint32_t d, uint32_t rest) {
    return 2 * SS + SS * d + (rest == 0 ? 0u : rest <= 4 ? 4u : 8u);
}

// Fused per-step parameters for the perception / update kernels.
struct StepParams {
    GridParams g;
    uint32_t N, B, S, H, F;
    uint32_t SS;    // sorted state row stride (state_stride_for(S))
    uint32_t FP;    // padded feature row width (padded_features)
    uint32_t T;     // total particles B*N (feature-major row count)
    uint32_t state_grad, density_grad, log_norm_grad, log_norm_dgrad, hybrid, position_features;
    float state_scale;  // normalize_state_gradient factor
    float dgrad_scale;  // normalize_density_gradient factor
    float alpha, motion_eps, dt;
    uint32_t gates3d;
    float update_prob;
    uint32_t step_index;
    uint32_t base_seed;
    uint32_t mlp_engine;  // NPA_MLP_VALU (bit-exact) or NPA_MLP_MFMA
    // cell directory of the split bins (set by the neighbour-pass launchers)
    const uint32_t* dir_n;
    const int4* dir_e;
};

struct StepIO {
    const float4* pos = nullptr;     // original order
    const float* states = nullptr;   // original order
    const float* mask = nullptr;     // optional, original order
    const float* w1 = nullptr;
    const float* b1 = nullptr;
    const float* w2 = nullptr;
    const float* b2 = nullptr;
    float4* out_pos = nullptr;
    float* out_states = nullptr;
    float* out_density = nullptr;    // optional
    // perceive-mode outputs
    float* features = nullptr;
    float* blurred = nullptr;
    float* state_gradient = nullptr;
    float* density_gradient = nullptr;
};

// The targets of a fused step: the caller's mask, else the device hash mask when update_prob < 1,
// else every particle.
inline SplitTargets step_targets(const StepParams& p, const StepIO& io) {
    SplitTargets t;
    t.mask_mode = io.mask ? 2 : (p.update_prob < 1.0f ? 1 : 0);
    t.mask = io.mask;
    t.update_prob = p.update_prob;
    t.step_index = p.step_index;
    t.base_seed = p.base_seed;
    t.pos = io.pos;
    t.states = io.states;
    t.out_pos = io.out_pos;
    t.out_states = io.out_states;
    return t;
}

// Density pass; then the perception pass writing feature rows (mode 0: sorted order into the
// workspace, followed by the MLP + Euler kernel; mode 1: the perceive outputs in original order),
// over the targets the hashgrid build selected.
hipError_t launch_density(const StepParams& p, Workspace& ws, float* density_out, int grid_blocks,
                          hipStream_t stream, Profiler* prof);
hipError_t launch_update(const StepParams& p, Workspace& ws, const StepIO& io, int mode,
                         int grid_blocks, hipStream_t stream, Profiler* prof);
// The second pass (and in mode 0 the MLP) of one dimension; launch_update runs them after the
// update-mask kernel. `blocks` = one wave per block.
hipError_t launch_second_pass_2d(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int blocks,
                                 hipStream_t stream, Profiler* prof);
hipError_t launch_second_pass_3d(const StepParams& p, Workspace& ws, const StepIO& io, int mode, int blocks,
                                 hipStream_t stream, Profiler* prof);
// Padded weights, two layouts one after the other in one buffer: the MLP kernel's w1t [FP][HP]
// (features at their padded positions), b1p [HP], w2t [H][OP] (transposed), b2p [OP]; then, at
// float offset valu_weight_floats(p), the fused update kernel's (fused_weight_floats(p)).
// Zeros everywhere else.
size_t padded_weight_floats(const StepParams& p);
size_t valu_weight_floats(const StepParams& p);
size_t fused_weight_floats(const StepParams& p);
hipError_t launch_pad_weights(const StepParams& p, const float* w1, const float* b1, const float* w2,
                              const float* b2, float* wpad, hipStream_t stream);
hipError_t launch_pad_weights_fused(const StepParams& p, const float* w1, const float* b1, const float* w2,
                                    const float* b2, float* wf, hipStream_t stream);
// The fused second pass + update MLP + Euler step (npa_update.hip) for 16-wide sorted rows,
// H <= 128, either MLP engine; wfused = the fused layout of the padded weights.
bool fused_update_applies(const StepParams& p);
hipError_t launch_update_fused_2d(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                  hipStream_t stream, Profiler* prof);
hipError_t launch_update_fused_3d(const StepParams& p, Workspace& ws, const StepIO& io, const float* wfused,
                                  hipStream_t stream, Profiler* prof);
hipError_t launch_mlp_forward(const StepParams& p, const float* features, uint32_t rows,
                              const StepIO& io, float* dx, float* ds, hipStream_t stream);
hipError_t launch_euler(const StepParams& p, const float4* pos, const float* states,
                        const float4* dx, const float* ds, const float* mask, float4* out_pos,
                        float* out_states, uint64_t total, hipStream_t stream);
hipError_t launch_update_mask(uint32_t batch, uint32_t n, float p, uint32_t step, uint32_t base_seed,
                              float* mask, hipStream_t stream);
hipError_t launch_count_pairs(const StepParams& p, Workspace& ws, int grid_blocks,
                              unsigned long long* counters, hipStream_t stream);
hipError_t launch_neighbor_lists(const StepParams& p, Workspace& ws, uint32_t* counts_or_offsets,
                                 uint32_t* indices, int write, int grid_blocks, hipStream_t stream);

// decode / splat
hipError_t launch_decode_gaussians(const float4* pos, const float* states, uint32_t count,
                                   uint32_t state_dims, const npa_gaussian_decode_cfg& cfg,
                                   float* pv, float* sh, float* rot, float* so, hipStream_t stream);
// write_gaussian_from_output (gpu_step.wgsl:4963-5052) of `total` particles: pv, rot, so [total][4],
// sh [total][NPA_GAUSSIAN_SH_COEFF_COUNT], all 16-byte aligned.
hipError_t launch_write_gaussians(const float4* pos, const float* states, uint32_t total, uint32_t particle_count,
                                  uint32_t S, uint32_t dim, float eps, bool position_features, float* pv, float* sh,
                                  float* rot, float* so, hipStream_t stream);
struct SplatWorkspace {
    DevBuf params, item_start, keys, vals, sorted, ranks, table, totals, offsets, count, flags, scan;
    DevBuf attrs;  // render attributes of a state's particles: colours [n][3], opacities [n], sigmas [n]
    DevBuf partials, chunks;  // render: per-chunk partial tiles; chunk counts, starts and total
    DevBuf order;      // oriented raster: depth order
    DevBuf sort_temp;  // oriented raster: the radix sort's temporary storage
    DevBuf decoded;  // oriented raster of a state: its decoded Gaussians
    void release();
};
// Particle n is drawn into window n / per_window of a grid of `windows` windows, win_cols per
// row, each cfg.image_size pixels square (one window: the plain splat).
hipError_t launch_splat_2d(const float4* pos, const float* colors, const float* states,
                           uint32_t state_dims, uint32_t count, const npa_splat2d_cfg& cfg,
                           float* image, SplatWorkspace& ws, hipStream_t stream, Profiler* prof,
                           uint32_t per_window, uint32_t windows, uint32_t win_cols);

// Projected 3D render (render_loss/projection.rs + image.rs): images[nviews][size][size][5].
// views is a host array of nviews <= kMaxRenderViews NPA_VIEW_* values.
constexpr uint32_t kMaxRenderViews = 16;
hipError_t launch_render_views(const float4* pos, const float* colors, const float* opacities,
                               const float* sigmas, uint32_t count, const uint32_t* views, uint32_t nviews,
                               const npa_render_cfg& cfg, float* images, SplatWorkspace& ws,
                               hipStream_t stream, Profiler* prof);
// Stable sort of the indices 0..n-1 by keys[i] (bits [0, end_bit)): order[k] is the index of
// the k-th smallest key, equal keys in ascending index; keys_out receives the sorted keys.
hipError_t sort_index_by_key(const uint32_t* keys, uint32_t* keys_out, uint32_t* order, uint32_t n,
                             uint32_t end_bit, DevBuf& temp, hipStream_t stream);
// EWA raster of oriented Gaussians (npa_raster_gaussians_3d): image[height][width][4]. Reads the
// (tile, Gaussian) item total back to the host (one stream synchronisation). coef_stride: the
// coefficient triples stored per Gaussian (0: (sh_degree + 1)^2, the camera's own count); a
// decode's colours in RGB mode are read from the first triple of each Gaussian's row.
hipError_t launch_raster_gaussians(const float4* position_visibility, const float* spherical_harmonic,
                                   const float4* rotation, const float4* scale_opacity, uint32_t count,
                                   const npa_raster_camera& cam, float* image, SplatWorkspace& ws,
                                   hipStream_t stream, Profiler* prof, uint32_t coef_stride = 0);
// state_tail_render_attributes (render_loss/attributes.rs:15-87); derivatives may be null.
hipError_t launch_render_attributes(const float* states, uint32_t count, uint32_t state_dims,
                                    const npa_render_cfg& cfg, float* colors, float* opacities,
                                    float* sigmas, float* derivatives, hipStream_t stream);

// Perception adjoint (reference/adjoint.rs): per-slot scratch of the four adjoint passes.
struct AdjointWorkspace {
    DevBuf sdens, sfb, rga, madj, rda, dadj, ppos;
    void release();
};
// Needs the hashgrid built with its payload (sorted records and states) in ws; fadj [T][F],
// state_adj [T][S] and pos_adj [T] in particle order.
hipError_t launch_perceive_adjoint(const StepParams& p, Workspace& ws, AdjointWorkspace& aw, const float* fadj,
                                   float* state_adj, float4* pos_adj, hipStream_t stream);

int device_cu_count();

// A kernel's dynamic-LDS limit, raised once per device to the 160 KiB a gfx950 workgroup can hold
// less the kernel's static LDS (each launch still asks for what it uses). Thread-safe: a device's
// flag is set only after the attribute call succeeded, and threads that race on a first launch all
// set the same value.
constexpr int kMaxLdsDevices = 64;
constexpr uint32_t kMaxLdsBytes = 163840;
struct LdsLimitFlags {
    std::atomic<bool> done[kMaxLdsDevices];
};
inline hipError_t raise_lds_limit(const void* fn, LdsLimitFlags& flags) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const bool tracked = dev >= 0 && dev < kMaxLdsDevices;
    if (tracked && flags.done[dev].load(std::memory_order_acquire)) return hipSuccess;
    hipFuncAttributes attr{};
    e = hipFuncGetAttributes(&attr, fn);
    if (e != hipSuccess) return e;
    const int dyn = (int)kMaxLdsBytes - (int)attr.sharedSizeBytes;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
    if (e == hipSuccess && tracked) flags.done[dev].store(true, std::memory_order_release);
    return e;
}

}  // namespace npa
