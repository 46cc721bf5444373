// npa_abi.cpp - the C ABI of libnpa_hip.so (declared in include/npa_abi.h).
//
// Validation mirrors the reference's error behaviour: HashGridConfig::validate
// (crates/burn_automata_kernels/src/config.rs:65-84), check_shapes
// (crates/burn_automata_kernels/src/reference/shape.rs:3-25), NpaModel::validate and the
// grid/model dim check of step_cpu (crates/burn_automata/src/model.rs:756-783).
#include <hip/hip_runtime.h>

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "npa_internal.hpp"

using npa::DevBuf;

struct npa_context {
    int device = 0;
    hipStream_t stream = nullptr;
    bool host_io = false;
    int mlp_engine = NPA_MLP_VALU;  // npa_step's update-MLP engine
    int cus = 256;
    std::string last_error;
    npa::Workspace ws;
    npa::SplatWorkspace splat_ws;
    npa::AdjointWorkspace adj_ws;
    npa::Profiler prof;
    std::vector<DevBuf*> staging;
    // npa_step_noalloc: this device's copy of the scratch array (null when it is unavailable, with
    // the reason in scratch_err) and a view of its flag words for npa_context_synchronize
    void* scratch = nullptr;
    hipError_t scratch_err = hipSuccess;
    npa::Workspace scratch_flags;
    // set by this context's first npa_step_noalloc call: only then does npa_context_synchronize read
    // the scratch array's flag words (which every context on the GPU shares)
    std::atomic<bool> used_noalloc{false};
    // the caller's handle plus one per live npa_state: a state keeps its context until it is destroyed
    std::atomic<int> refs{1};
    ~npa_context() {
        ws.release();
        splat_ws.release();
        adj_ws.release();
        for (DevBuf* b : staging) {
            b->release();
            delete b;
        }
    }
};

struct npa_state {
    npa_context* ctx = nullptr;
    npa_model_cfg model{};
    npa_grid_cfg grid{};
    uint32_t B = 0, N = 0;
    float dt = 1.0f, update_prob = 1.0f;
    uint64_t seed = 0;
    uint64_t step_index = 0;
    int mlp_engine = NPA_MLP_VALU;
    DevBuf pos[2], states[2], density, w1, b1, w2, b2;
    int cur = 0;
    npa::Workspace ws;
    npa::SplatWorkspace splat_ws;
    npa::HashgridPlan plan;
    int grid_blocks = 1;
    ~npa_state() {
        for (DevBuf* b : {&pos[0], &pos[1], &states[0], &states[1], &density, &w1, &b1, &w2, &b2}) b->release();
        ws.release();
        splat_ws.release();
    }
};

namespace {

npa_status fail(npa_context* ctx, npa_status st, const std::string& msg) {
    if (ctx) ctx->last_error = msg;
    return st;
}

npa_status hip_fail(npa_context* ctx, hipError_t e, const char* where) {
    std::string msg = std::string(where) + ": " + hipGetErrorString(e);
    return fail(ctx, e == hipErrorOutOfMemory ? NPA_ERR_OUT_OF_MEMORY : NPA_ERR_DEVICE, msg);
}

#define NPA_HIP(ctx, expr, where)                          \
    do {                                                   \
        hipError_t _e = (expr);                            \
        if (_e != hipSuccess) return hip_fail(ctx, _e, where); \
    } while (0)

std::string fmt_f(float v) {
    char buf[64];
    snprintf(buf, sizeof buf, "%g", (double)v);
    return buf;
}

// HashGridConfig::validate  config.rs:65-84
npa_status validate_grid(npa_context* ctx, const npa_grid_cfg* cfg) {
    if (!cfg) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null grid config");
    if (!(cfg->dim == 2 || cfg->dim == 3))
        return fail(ctx, NPA_ERR_INVALID_DIM, "expected spatial dim 2 or 3, got " + std::to_string(cfg->dim));
    if (!std::isfinite(cfg->eps) || cfg->eps <= 0.0f)
        return fail(ctx, NPA_ERR_INVALID_EPS, "eps must be finite and positive, got " + fmt_f(cfg->eps));
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        const uint32_t s = cfg->grid_size[a];
        if (s == 0) return fail(ctx, NPA_ERR_INVALID_GRID_SIZE, "grid sizes must be non-zero for active dimensions");
        if (cfg->mode == NPA_MODE_PARTICLE && (s & (s - 1u)) != 0)
            return fail(ctx, NPA_ERR_PARTICLE_MODE_POW2,
                        "particle hashgrid mode requires power-of-two grid size at axis " + std::to_string(a) +
                            ", got " + std::to_string(s));
    }
    if (cfg->boundary > 1 || cfg->mode > 1)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: unknown boundary or hashgrid mode");
    return NPA_OK;
}

npa_status check_model(npa_context* ctx, const npa_model_cfg* m, const npa_grid_cfg* grid) {
    if (!m) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null model config");
    if (!(m->spatial_dims == 2 || m->spatial_dims == 3))
        return fail(ctx, NPA_ERR_INVALID_MODEL,
                    "invalid model: spatial_dims must be 2 or 3, got " + std::to_string(m->spatial_dims));
    if (grid && grid->dim != m->spatial_dims)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: grid dim " + std::to_string(grid->dim) + " does not match model spatial dims " +
                        std::to_string(m->spatial_dims));
    if (m->state_dims == 0 || m->state_dims > 32)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: the device path supports 1..=32 state dims, got " + std::to_string(m->state_dims));
    if (m->equivariance > 2) return fail(ctx, NPA_ERR_INVALID_MODEL, "invalid model: unknown equivariance mode");
    if (m->spatial_dims == 3 && m->position_features && m->state_dims > 3 && m->state_dims < 8)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: position-conditioned 3D gates read state channel 7; need state_dims >= 8");
    return NPA_OK;
}

uint32_t model_perception_dims(const npa_model_cfg& m) {  // config.rs:133-139
    return m.state_dims * 2 + (m.state_grad ? m.state_dims * m.spatial_dims : 0) +
           (m.density_grad ? m.spatial_dims : 0) + (m.position_features ? m.spatial_dims : 0);
}

npa_perception_opts opts_for_model(const npa_model_cfg& m) {  // model.rs:784-800
    npa_perception_opts o{};
    o.state_grad = m.state_grad;
    o.density_grad = m.density_grad;
    o.eps0 = m.eps0;
    o.scale_equivariance = m.equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE;
    o.particle_density_equivariance =
        m.equivariance == NPA_EQUIV_PARTICLE_DENSITY || m.equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE;
    o.log_norm_grad = m.log_norm_grad;
    o.log_norm_density_grad = m.log_norm_density_grad;
    o.hybrid_state_gradient = 1;
    o.position_features = m.position_features;
    return o;
}

npa::StepParams make_params(const npa_grid_cfg& cfg, const npa_perception_opts& o, uint32_t B, uint32_t N,
                            uint32_t S) {
    npa::StepParams p{};
    p.g = npa::make_grid_params(cfg);
    p.g.spatial = cfg.mode == NPA_MODE_PARTICLE ? 1 : 0;  // the step's own sort: coordinate bins
    p.N = N;
    p.B = B;
    p.S = S;
    p.state_grad = o.state_grad ? 1 : 0;
    p.density_grad = o.density_grad ? 1 : 0;
    p.log_norm_grad = o.log_norm_grad ? 1 : 0;
    p.log_norm_dgrad = o.log_norm_density_grad ? 1 : 0;
    p.hybrid = o.hybrid_state_gradient ? 1 : 0;
    p.position_features = o.position_features ? 1 : 0;
    p.F = S * 2 + (o.state_grad ? S * cfg.dim : 0) + (o.density_grad ? cfg.dim : 0) +
          (o.position_features ? cfg.dim : 0);
    p.SS = npa::state_stride_for(S);
    p.FP = npa::padded_features(p.SS, cfg.dim,
                                (o.density_grad ? cfg.dim : 0) + (o.position_features ? cfg.dim : 0));
    p.T = B * N;
    // normalize_state_gradient / normalize_density_gradient  normalize.rs:5-58
    const float eps0 = fmaxf(o.eps0, FLT_MIN);
    p.state_scale = o.scale_equivariance ? cfg.eps / eps0 : 1.0f;
    const float s1 = o.scale_equivariance ? npa::host_powi(cfg.eps / eps0, 1 + (int)cfg.dim) : 1.0f;
    const float s2 = o.particle_density_equivariance ? 1.0f / (float)(N > 1 ? N : 1) : 1.0f;
    p.dgrad_scale = s1 * s2;
    p.update_prob = 1.0f;
    p.dt = 1.0f;
    return p;
}

void apply_model(npa::StepParams* p, const npa_model_cfg& m, float grid_eps) {
    p->H = m.hidden_dims;
    p->alpha = m.alpha;
    // NpaConfig::motion_eps  config.rs:156-162
    p->motion_eps = m.equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE ? grid_eps : m.eps0;
    p->gates3d = (m.spatial_dims == 3 && m.position_features && m.state_dims > 3) ? 1 : 0;
}

uint32_t base_seed(uint64_t seed) { return (uint32_t)seed ^ (uint32_t)(seed >> 32); }  // params.rs:186-188

int grid_blocks_for(const npa_context* ctx, const npa::HashgridPlan& plan) {
    const uint64_t waves = plan.worklist_cap;
    const uint64_t blocks = (waves + 3) / 4;
    const uint64_t cap = (uint64_t)ctx->cus * 8;
    return (int)std::max<uint64_t>(1, std::min(blocks, cap));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ------------------------------------------------------------ no-allocation workspace
// npa_step_noalloc's workspace: a file-scope device array, one copy per GPU (each at its own
// address), held until the process ends. In host code `scratch` is only a stand-in for the symbol,
// not a device address: it is never passed to a kernel or a copy. Set-up resolves each device's
// address with hipGetSymbolAddress (with that device current) and everything uses that address.
static __device__ __align__(256) unsigned char scratch[NPA_STEP_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
bool g_scratch_done[kMaxScratchDevices] = {};
void* g_scratch_ptr[kMaxScratchDevices] = {};
hipError_t g_scratch_err[kMaxScratchDevices] = {};

// Once per device (the current one): the device address of `scratch`, with its flag words cleared.
hipError_t scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_done[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess) {
            static const uint32_t zero[npa::kCarveFlagBytes / 4] = {};
            e = hipMemcpy(p, zero, sizeof zero, hipMemcpyHostToDevice);
        }
        g_scratch_done[device] = true;
        g_scratch_err[device] = e;
        g_scratch_ptr[device] = e == hipSuccess ? p : nullptr;
    }
    *out = g_scratch_ptr[device];
    return g_scratch_err[device];
}

// Clears the first n (<= 64) words of a buffer (a kernel rather than a memset node, so that a
// caller may capture it in a graph).
__global__ void k_clear_words(uint32_t* __restrict__ words, uint32_t n) {
    if (threadIdx.x < n) words[threadIdx.x] = 0u;
}

// A null array that the call reads or writes is a caller error, refused before any HIP call
// (a null pointer would otherwise reach a kernel).
npa_status need(npa_context* ctx, std::initializer_list<const void*> arrays, const char* what) {
    for (const void* a : arrays)
        if (!a) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, std::string("invalid argument: null ") + what);
    return NPA_OK;
}

// The weight arrays of a model with F features, H hidden units and O outputs (empty ones may be null).
npa_status need_weights(npa_context* ctx, const npa_weights* w, uint64_t F, uint64_t H, uint64_t O) {
    if (!w) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null weights");
    if ((H * F && !w->w1) || (H && !w->b1) || (O * H && !w->w2) || (O && !w->b2))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null weight array");
    return NPA_OK;
}

// Host I/O: stages host arrays through context-owned device buffers.
struct HostIO {
    npa_context* ctx;
    bool active;
    size_t slot = 0;
    struct Out { void* host; void* dev; size_t bytes; };
    std::vector<Out> outs;
    hipError_t err = hipSuccess;
    explicit HostIO(npa_context* c) : ctx(c), active(c->host_io) {}
    void* buffer(size_t bytes) {
        if (slot == ctx->staging.size()) ctx->staging.push_back(new DevBuf());
        DevBuf* b = ctx->staging[slot++];
        hipError_t e = b->reserve(bytes ? bytes : 16);
        if (e != hipSuccess) {
            err = e;
            return nullptr;
        }
        return b->ptr;
    }
    template <class T>
    const T* in(const T* p, size_t bytes) {
        if (!active || !p) return p;
        void* d = buffer(bytes);
        if (!d) return nullptr;
        if (bytes) {
            hipError_t e = hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, ctx->stream);
            if (e != hipSuccess) err = e;
        }
        return static_cast<const T*>(d);
    }
    template <class T>
    T* out(T* p, size_t bytes) {
        if (!active || !p) return p;
        void* d = buffer(bytes);
        if (!d) return nullptr;
        outs.push_back({(void*)p, d, bytes});
        return static_cast<T*>(d);
    }
    hipError_t finish() {
        if (err != hipSuccess) return err;
        if (!active) return hipSuccess;
        for (const Out& o : outs) {
            if (!o.bytes) continue;
            hipError_t e = hipMemcpyAsync(o.host, o.dev, o.bytes, hipMemcpyDeviceToHost, ctx->stream);
            if (e != hipSuccess) return e;
        }
        return hipStreamSynchronize(ctx->stream);
    }
};

// Reports (and clears) the coordinate overflows of every hashgrid build on `ws` since the last
// report: device-pointer calls queue their builds without waiting, so their overflow surfaces at
// the next call that synchronises (host-I/O calls, npa_neighbor_lists, npa_state_read,
// npa_context_synchronize).
npa_status check_flags(npa_context* ctx, npa::Workspace& ws) {
    if (!ws.flags.ptr) return NPA_OK;
    uint32_t flags[2] = {0, 0};
    NPA_HIP(ctx, hipMemcpyAsync(flags, ws.flags.ptr, 8, hipMemcpyDeviceToHost, ctx->stream), "flags readback");
    NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "flags readback");
    if ((flags[0] | flags[1]) & 1u) {
        const uint32_t zero[2] = {0, 0};
        NPA_HIP(ctx, hipMemcpyAsync(ws.flags.ptr, zero, 8, hipMemcpyHostToDevice, ctx->stream), "flags reset");
        NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "flags reset");
        return fail(ctx, NPA_ERR_COORD_OVERFLOW,
                    "a particle-mode cell coordinate left the +-2^30 range the device path stores exactly");
    }
    return NPA_OK;
}

npa_status set_device(npa_context* ctx) {
    NPA_HIP(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    return NPA_OK;
}

}  // namespace

// ====================================================================== context
extern "C" {

const char* npa_version(void) { return "npa_hip 0.1.0 (gfx950)"; }

npa_status npa_context_create(int device, void* stream, npa_context** out) {
    if (!out) return NPA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return NPA_ERR_DEVICE;
    if (device < 0 || device >= count) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = new npa_context();
    ctx->device = device;
    ctx->stream = (hipStream_t)stream;
    if (hipSetDevice(device) != hipSuccess) {
        delete ctx;
        return NPA_ERR_DEVICE;
    }
    ctx->cus = npa::device_cu_count();
    ctx->scratch_err = scratch_address(device, &ctx->scratch);
    if (ctx->scratch) ctx->scratch_flags.flags.view(ctx->scratch, npa::kCarveFlagBytes);
    *out = ctx;
    return NPA_OK;
}

namespace {
// Drops one reference; the last one waits for the context's queued work and frees it.
void context_release(npa_context* ctx) {
    if (ctx->refs.fetch_sub(1) != 1) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    delete ctx;
}
}  // namespace

void npa_context_destroy(npa_context* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    context_release(ctx);
}

npa_status npa_context_set_stream(npa_context* ctx, void* stream) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    ctx->stream = (hipStream_t)stream;
    return NPA_OK;
}

npa_status npa_context_set_host_io(npa_context* ctx, int host_io) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    ctx->host_io = host_io != 0;
    return NPA_OK;
}

namespace {
// Width of the feature-major rows a step's workspace holds: none when the fused second pass + MLP
// kernel runs the step (its feature rows never leave LDS).
uint32_t feature_rows_for(const npa::StepParams& p) { return npa::fused_update_applies(p) ? 0u : p.FP; }
}  // namespace

npa_status npa_context_set_mlp_engine(npa_context* ctx, int engine) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    if (engine != NPA_MLP_VALU && engine != NPA_MLP_MFMA && engine != NPA_MLP_MFMA_BF16)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: unknown MLP engine " + std::to_string(engine));
    ctx->mlp_engine = engine;
    return NPA_OK;
}

npa_status npa_context_synchronize(npa_context* ctx) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    npa_status st = check_flags(ctx, ctx->ws);
    if (st) return st;
    // the no-allocation step's overflow word is per GPU, not per context: a context that never called
    // npa_step_noalloc neither reads nor clears it
    if (!ctx->used_noalloc.load(std::memory_order_relaxed)) return NPA_OK;
    return check_flags(ctx, ctx->scratch_flags);
}

const char* npa_last_error(const npa_context* ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }

// ============================================================== operator surface
npa_status npa_build_hashgrid(npa_context* ctx, const float* positions, uint32_t B, uint32_t N,
                              const npa_grid_cfg* cfg, uint32_t* bin_offsets, size_t bin_offsets_len,
                              uint32_t* permutation, uint32_t* inverse_permutation, size_t particles_len) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, cfg);
    if (st) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t total = (uint64_t)B * N;
    uint64_t cells = 1;
    for (uint32_t a = 0; a < cfg->dim; ++a) cells *= cfg->grid_size[a];
    if (bin_offsets_len != (uint64_t)B * cells + 1)
        return fail(ctx, NPA_ERR_OUTPUT_SHAPE,
                    "output buffer length " + std::to_string(bin_offsets_len) + " does not match expected " +
                        std::to_string((uint64_t)B * cells + 1));
    if (particles_len != total)
        return fail(ctx, NPA_ERR_OUTPUT_SHAPE,
                    "output buffer length " + std::to_string(particles_len) + " does not match expected " +
                        std::to_string(total));
    if (!positions && total) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null positions");
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*cfg, B, N, &plan, &err)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, total * 16);
    uint32_t* bo = io.out(bin_offsets, bin_offsets_len * 4);
    uint32_t* perm = io.out(permutation, total * 4);
    uint32_t* inv = io.out(inverse_permutation, total * 4);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (total && !aligned16(pos)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions must be 16-byte aligned");
    NPA_HIP(ctx, ctx->ws.reserve(plan, total, B, 1, (int)cfg->dim), "workspace");
    const npa::GridParams g = npa::make_grid_params(*cfg);
    if (total) {
        NPA_HIP(ctx, npa::launch_hashgrid(plan, g, pos, nullptr, 1, B, N, ctx->ws, false, ctx->stream, &ctx->prof),
                "hashgrid");
        NPA_HIP(ctx, hipMemcpyAsync(bo, ctx->ws.bin_offsets.ptr, bin_offsets_len * 4, hipMemcpyDeviceToDevice, ctx->stream),
                "copy bin_offsets");
        NPA_HIP(ctx, hipMemcpyAsync(perm, ctx->ws.perm.ptr, total * 4, hipMemcpyDeviceToDevice, ctx->stream), "copy perm");
        NPA_HIP(ctx, hipMemcpyAsync(inv, ctx->ws.inv.ptr, total * 4, hipMemcpyDeviceToDevice, ctx->stream), "copy inv");
    } else {
        NPA_HIP(ctx, hipMemsetAsync(bo, 0, bin_offsets_len * 4, ctx->stream), "zero bin_offsets");
    }
    NPA_HIP(ctx, io.finish(), "host io");
    if (ctx->host_io) return check_flags(ctx, ctx->ws);
    return NPA_OK;
}

npa_status npa_neighbor_lists(npa_context* ctx, const float* positions, uint32_t B, uint32_t N,
                              const npa_grid_cfg* cfg, uint32_t* offsets, uint32_t* indices, size_t capacity,
                              size_t* required) {
    if (!ctx || !offsets || !required) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, cfg);
    if (st) return st;
    const uint64_t total = (uint64_t)B * N;
    if (total && (st = need(ctx, {positions}, "positions"))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*cfg, B, N, &plan, &err)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, total * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    NPA_HIP(ctx, ctx->ws.reserve(plan, total, B, 1, (int)cfg->dim), "workspace");
    npa_perception_opts o{};
    npa::StepParams p = make_params(*cfg, o, B, N, 1);
    const int blocks = grid_blocks_for(ctx, plan);
    std::vector<uint32_t> counts(total + 1, 0);
    DevBuf dcounts;
    NPA_HIP(ctx, dcounts.reserve((total + 1) * 4), "counts");
    if (total) {
        NPA_HIP(ctx, npa::launch_hashgrid(plan, p.g, pos, nullptr, 1, B, N, ctx->ws, true, ctx->stream, nullptr),
                "hashgrid");
        NPA_HIP(ctx, npa::launch_neighbor_lists(p, ctx->ws, dcounts.as<uint32_t>(), nullptr, 0, blocks, ctx->stream),
                "count");
        NPA_HIP(ctx, hipMemcpyAsync(counts.data(), dcounts.ptr, total * 4, hipMemcpyDeviceToHost, ctx->stream),
                "counts readback");
        NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "sync");
    }
    std::vector<uint32_t> off(total + 1, 0);
    for (uint64_t i = 0; i < total; ++i) off[i + 1] = off[i] + counts[i];
    *required = off[total];
    if (ctx->host_io) {
        memcpy(offsets, off.data(), (total + 1) * 4);
    } else {
        NPA_HIP(ctx, hipMemcpy(offsets, off.data(), (total + 1) * 4, hipMemcpyHostToDevice), "offsets");
    }
    if (indices && capacity >= off[total] && total) {
        NPA_HIP(ctx, hipMemcpy(dcounts.ptr, off.data(), total * 4, hipMemcpyHostToDevice), "offsets upload");
        DevBuf didx;
        uint32_t* dst = indices;
        if (ctx->host_io) {
            NPA_HIP(ctx, didx.reserve((size_t)off[total] * 4 + 4), "indices");
            dst = didx.as<uint32_t>();
        }
        NPA_HIP(ctx, npa::launch_neighbor_lists(p, ctx->ws, dcounts.as<uint32_t>(), dst, 1, blocks, ctx->stream),
                "fill");
        if (ctx->host_io)
            NPA_HIP(ctx, hipMemcpyAsync(indices, dst, (size_t)off[total] * 4, hipMemcpyDeviceToHost, ctx->stream),
                    "indices readback");
        NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "sync");
        didx.release();
    }
    dcounts.release();
    return check_flags(ctx, ctx->ws);
}

npa_status npa_perceive(npa_context* ctx, const float* positions, const float* states, uint32_t B, uint32_t N,
                        uint32_t S, const npa_grid_cfg* cfg, const npa_perception_opts* opts, float* features,
                        size_t features_len, float* density, float* blurred_state, float* state_gradient,
                        float* density_gradient, uint32_t* feature_dims) {
    if (!ctx || !opts) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, cfg);
    if (st) return st;
    if (S == 0 || S > 32)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: the device path supports 1..=32 state dims");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t total = (uint64_t)B * N;
    const uint32_t d = cfg->dim;
    const uint32_t F = S * 2 + (opts->state_grad ? S * d : 0) + (opts->density_grad ? d : 0) +
                       (opts->position_features ? d : 0);
    if (feature_dims) *feature_dims = F;
    if (features_len != total * F)
        return fail(ctx, NPA_ERR_OUTPUT_SHAPE,
                    "output buffer length " + std::to_string(features_len) + " does not match expected " +
                        std::to_string(total * F));
    if (!features || !density || (total && (!positions || !states)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null array");
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*cfg, B, N, &plan, &err))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, total * 16);
    const float* st_in = io.in(states, total * S * 4);
    npa::StepIO sio;
    sio.pos = pos;
    sio.states = st_in;
    sio.features = io.out(features, total * F * 4);
    float* dens = io.out(density, total * 4);
    sio.blurred = io.out(blurred_state, total * S * 4);
    sio.state_gradient = opts->state_grad ? io.out(state_gradient, total * S * d * 4) : nullptr;
    sio.density_gradient = opts->density_grad ? io.out(density_gradient, total * d * 4) : nullptr;
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (total && !aligned16(pos)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions must be 16-byte aligned");
    if (total && (S % 4 == 0) && !aligned16(st_in))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: states must be 16-byte aligned");
    NPA_HIP(ctx, ctx->ws.reserve(plan, total, B, S, (int)d), "workspace");
    npa::StepParams p = make_params(*cfg, *opts, B, N, S);
    const int blocks = grid_blocks_for(ctx, plan);
    if (total) {
        NPA_HIP(ctx, npa::launch_hashgrid(plan, p.g, pos, st_in, S, B, N, ctx->ws, true, ctx->stream, &ctx->prof),
                "hashgrid");
        NPA_HIP(ctx, npa::launch_density(p, ctx->ws, dens, blocks, ctx->stream, &ctx->prof), "density");
        NPA_HIP(ctx, npa::launch_update(p, ctx->ws, sio, 1, blocks, ctx->stream, &ctx->prof), "perceive");
    }
    NPA_HIP(ctx, io.finish(), "host io");
    if (ctx->host_io) return check_flags(ctx, ctx->ws);
    return NPA_OK;
}

npa_status npa_perceive_adjoint(npa_context* ctx, const float* positions, const float* states, uint32_t B,
                                uint32_t N, uint32_t S, const npa_grid_cfg* cfg, const npa_perception_opts* opts,
                                const float* feature_adjoint, size_t feature_adjoint_len, float* state_adjoint,
                                float* position_adjoint) {
    if (!ctx || !opts) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, cfg);
    if (st) return st;
    if (S == 0 || S > 32)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: the device path supports 1..=32 state dims");
    const uint64_t total = (uint64_t)B * N;
    const uint32_t d = cfg->dim;
    const uint32_t F = S * 2 + (opts->state_grad ? S * d : 0) + (opts->density_grad ? d : 0) +
                       (opts->position_features ? d : 0);
    if (feature_adjoint_len != total * F)  // adjoint.rs:48-54
        return fail(ctx, NPA_ERR_OUTPUT_SHAPE,
                    "output buffer length " + std::to_string(feature_adjoint_len) + " does not match expected " +
                        std::to_string(total * F));
    if (!state_adjoint || (total && (!positions || !states || !feature_adjoint)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null array");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*cfg, B, N, &plan, &err))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, total * 16);
    const float* st_in = io.in(states, total * S * 4);
    const float* fa = io.in(feature_adjoint, total * F * 4);
    float* sa = io.out(state_adjoint, total * S * 4);
    DevBuf pos_scratch;  // the position adjoint is computed even when the caller does not want it
    float4* pa = (float4*)(position_adjoint ? io.out(position_adjoint, total * 16) : nullptr);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!pa) {
        NPA_HIP(ctx, pos_scratch.reserve(total * 16 + 16), "workspace");
        pa = pos_scratch.as<float4>();
    }
    if (total && (!aligned16(pos) || !aligned16(pa)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: position arrays must be 16-byte aligned");
    NPA_HIP(ctx, ctx->ws.reserve(plan, total, B, S, (int)d), "workspace");
    npa::StepParams p = make_params(*cfg, *opts, B, N, S);
    if (total) {
        NPA_HIP(ctx, npa::launch_hashgrid(plan, p.g, pos, st_in, S, B, N, ctx->ws, true, ctx->stream, &ctx->prof),
                "hashgrid");
        NPA_HIP(ctx, npa::launch_perceive_adjoint(p, ctx->ws, ctx->adj_ws, fa, sa, pa, ctx->stream), "adjoint");
    }
    NPA_HIP(ctx, io.finish(), "host io");
    if (!position_adjoint) {
        NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "sync");
        pos_scratch.release();
    }
    if (ctx->host_io) return check_flags(ctx, ctx->ws);
    return NPA_OK;
}

npa_status npa_mlp_forward(npa_context* ctx, const float* features, uint32_t rows, const npa_model_cfg* model,
                           const npa_weights* w, float eps, float* dx, float* ds) {
    if (!ctx || !w) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_model(ctx, model, nullptr);
    if (st) return st;
    const uint32_t F = model_perception_dims(*model), H = model->hidden_dims, S = model->state_dims;
    const uint32_t O = model->spatial_dims + S;
    if (rows && (st = need(ctx, {features, dx, ds}, "features or outputs"))) return st;
    if ((st = need_weights(ctx, w, F, H, O))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    npa::StepIO sio;
    const float* f = io.in(features, (uint64_t)rows * F * 4);
    sio.w1 = io.in(w->w1, (uint64_t)H * F * 4);
    sio.b1 = io.in(w->b1, (uint64_t)H * 4);
    sio.w2 = io.in(w->w2, (uint64_t)O * H * 4);
    sio.b2 = io.in(w->b2, (uint64_t)O * 4);
    float* ddx = io.out(dx, (uint64_t)rows * 16);
    float* dds = io.out(ds, (uint64_t)rows * S * 4);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    npa_grid_cfg gcfg{};
    gcfg.dim = model->spatial_dims;
    gcfg.eps = eps;
    for (int a = 0; a < 3; ++a) gcfg.grid_size[a] = 1;
    npa::StepParams p = make_params(gcfg, opts_for_model(*model), 1, rows ? rows : 1, S);
    apply_model(&p, *model, eps);
    p.F = F;
    NPA_HIP(ctx, npa::launch_mlp_forward(p, f, rows, sio, ddx, dds, ctx->stream), "mlp");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_euler_step(npa_context* ctx, const float* positions, const float* states, const float* dx,
                          const float* ds, uint32_t B, uint32_t N, uint32_t S, const npa_grid_cfg* cfg, float dt,
                          const float* mask, float* out_positions, float* out_states) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, cfg);
    if (st) return st;
    const uint64_t total = (uint64_t)B * N;
    if (total && (st = need(ctx, {positions, states, dx, ds, out_positions, out_states}, "input or output array")))
        return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, total * 16);
    const float* sin_ = io.in(states, total * S * 4);
    const float4* ddx = (const float4*)io.in(dx, total * 16);
    const float* dds = io.in(ds, total * S * 4);
    const float* m = io.in(mask, total * 4);
    float4* op = (float4*)io.out(out_positions, total * 16);
    float* os = io.out(out_states, total * S * 4);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (total && (!aligned16(pos) || !aligned16(ddx) || !aligned16(op)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: position arrays must be 16-byte aligned");
    npa_perception_opts o{};
    npa::StepParams p = make_params(*cfg, o, B, N ? N : 1, S);
    p.dt = dt;
    NPA_HIP(ctx, npa::launch_euler(p, pos, sin_, ddx, dds, m, op, os, total, ctx->stream), "euler");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_step(npa_context* ctx, const float* positions, const float* states, uint32_t B, uint32_t N,
                    const npa_grid_cfg* grid, const npa_model_cfg* model, const npa_weights* w, float dt,
                    const float* mask, float* out_positions, float* out_states, float* out_density) {
    if (!ctx || !w) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, grid);
    if (st) return st;
    if ((st = check_model(ctx, model, grid))) return st;
    const uint64_t total = (uint64_t)B * N;
    const uint32_t S = model->state_dims, F = model_perception_dims(*model), H = model->hidden_dims;
    const uint32_t O = model->spatial_dims + S;
    if (total && (st = need(ctx, {positions, states, out_positions, out_states}, "positions, states or outputs")))
        return st;
    if ((st = need_weights(ctx, w, F, H, O))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*grid, B, N, &plan, &err))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    HostIO io(ctx);
    npa::StepIO sio;
    sio.pos = (const float4*)io.in(positions, total * 16);
    sio.states = io.in(states, total * S * 4);
    sio.mask = io.in(mask, total * 4);
    sio.w1 = io.in(w->w1, (uint64_t)H * F * 4);
    sio.b1 = io.in(w->b1, (uint64_t)H * 4);
    sio.w2 = io.in(w->w2, (uint64_t)O * H * 4);
    sio.b2 = io.in(w->b2, (uint64_t)O * 4);
    sio.out_pos = (float4*)io.out(out_positions, total * 16);
    sio.out_states = io.out(out_states, total * S * 4);
    float* dens = io.out(out_density, total * 4);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (total && (!aligned16(sio.pos) || !aligned16(sio.out_pos)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions must be 16-byte aligned");
    if (total && (S % 4 == 0) && !aligned16(sio.states))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: states must be 16-byte aligned");
    npa::StepParams p = make_params(*grid, opts_for_model(*model), B, N, S);
    apply_model(&p, *model, grid->eps);
    p.dt = dt;
    p.update_prob = 1.0f;
    p.mlp_engine = (uint32_t)ctx->mlp_engine;
    if (total && npa::state_stride_for(S) == S && !aligned16(sio.out_states))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: output states must be 16-byte aligned");
    NPA_HIP(ctx, ctx->ws.reserve(plan, total, B, S, (int)grid->dim, feature_rows_for(p)), "workspace");
    NPA_HIP(ctx, ctx->ws.wpad.reserve(npa::padded_weight_floats(p) * 4), "workspace");
    const int blocks = grid_blocks_for(ctx, plan);
    if (total) {
        NPA_HIP(ctx, npa::launch_pad_weights(p, sio.w1, sio.b1, sio.w2, sio.b2, ctx->ws.wpad.as<float>(), ctx->stream),
                "pad weights");
        const npa::SplitTargets targets = npa::step_targets(p, sio);
        NPA_HIP(ctx, npa::launch_hashgrid(plan, p.g, sio.pos, sio.states, S, B, N, ctx->ws, true, ctx->stream,
                                          &ctx->prof, &targets),
                "hashgrid");
        NPA_HIP(ctx, npa::launch_density(p, ctx->ws, dens, blocks, ctx->stream, &ctx->prof), "density");
        NPA_HIP(ctx, npa::launch_update(p, ctx->ws, sio, 0, blocks, ctx->stream, &ctx->prof), "update");
    }
    NPA_HIP(ctx, io.finish(), "host io");
    if (ctx->host_io) return check_flags(ctx, ctx->ws);
    return NPA_OK;
}

npa_status npa_step_noalloc(npa_context* ctx, const float* positions, const float* states, uint32_t B, uint32_t N,
                            const npa_grid_cfg* grid, const npa_model_cfg* model, const npa_weights* w, float dt,
                            const float* mask, float* out_positions, float* out_states, float* out_density) {
    if (!ctx || !w) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = validate_grid(ctx, grid);
    if (st) return st;
    if ((st = check_model(ctx, model, grid))) return st;
    const uint64_t total = (uint64_t)B * N;
    const uint32_t S = model->state_dims, F = model_perception_dims(*model), H = model->hidden_dims;
    const uint32_t O = model->spatial_dims + S;
    if (total && (st = need(ctx, {positions, states, out_positions, out_states}, "positions, states or outputs")))
        return st;
    if ((st = need_weights(ctx, w, F, H, O))) return st;
    if (ctx->host_io)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: npa_step_noalloc takes device pointers (host-I/O mode stages through "
                    "allocations)");
    if (!ctx->scratch)
        return fail(ctx, NPA_ERR_DEVICE,
                    std::string("no-allocation workspace unavailable: ") + hipGetErrorString(ctx->scratch_err));
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*grid, B, N, &plan, &err))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    npa::StepParams p = make_params(*grid, opts_for_model(*model), B, N, S);
    apply_model(&p, *model, grid->eps);
    p.dt = dt;
    p.update_prob = 1.0f;
    p.mlp_engine = (uint32_t)ctx->mlp_engine;
    npa::Workspace ws;  // views into this device's scratch array
    const uint64_t need_bytes = ws.carve(plan, total, B, S, (int)grid->dim, feature_rows_for(p),
                                         npa::padded_weight_floats(p) * 4,
                                         ctx->scratch, NPA_STEP_NOALLOC_SCRATCH_BYTES);
    if (need_bytes > NPA_STEP_NOALLOC_SCRATCH_BYTES)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: this system needs " + std::to_string(need_bytes) +
                        " bytes of workspace, above npa_step_noalloc's fixed " +
                        std::to_string((uint64_t)NPA_STEP_NOALLOC_SCRATCH_BYTES));
    if (total && (!aligned16(positions) || !aligned16(out_positions)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions must be 16-byte aligned");
    if (total && (S % 4 == 0) && !aligned16(states))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: states must be 16-byte aligned");
    if (total && npa::state_stride_for(S) == S && !aligned16(out_states))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: output states must be 16-byte aligned");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    if (!total) return NPA_OK;
    ctx->used_noalloc.store(true, std::memory_order_relaxed);
    npa::StepIO sio;
    sio.pos = (const float4*)positions;
    sio.states = states;
    sio.mask = mask;
    sio.w1 = w->w1;
    sio.b1 = w->b1;
    sio.w2 = w->w2;
    sio.b2 = w->b2;
    sio.out_pos = (float4*)out_positions;
    sio.out_states = out_states;
    const int blocks = grid_blocks_for(ctx, plan);
    // the build's overflow word must start at zero; everything else is written before it is read
    hipLaunchKernelGGL(k_clear_words, dim3(1), dim3(64), 0, ctx->stream, ws.flags.as<uint32_t>(), 1u);
    NPA_HIP(ctx, hipGetLastError(), "clear flags");
    NPA_HIP(ctx, npa::launch_pad_weights(p, sio.w1, sio.b1, sio.w2, sio.b2, ws.wpad.as<float>(), ctx->stream),
            "pad weights");
    const npa::SplitTargets targets = npa::step_targets(p, sio);
    NPA_HIP(ctx, npa::launch_hashgrid(plan, p.g, sio.pos, sio.states, S, B, N, ws, true, ctx->stream, nullptr, &targets),
            "hashgrid");
    NPA_HIP(ctx, npa::launch_density(p, ws, out_density, blocks, ctx->stream, nullptr), "density");
    NPA_HIP(ctx, npa::launch_update(p, ws, sio, 0, blocks, ctx->stream, nullptr), "update");
    return NPA_OK;
}

npa_status npa_update_mask(npa_context* ctx, uint32_t B, uint32_t N, float update_prob, uint32_t step_index,
                           uint64_t seed, float* mask) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = NPA_OK;
    if ((uint64_t)B * N && (st = need(ctx, {mask}, "mask"))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    float* m = io.out(mask, (uint64_t)B * N * 4);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    NPA_HIP(ctx, npa::launch_update_mask(B, N, update_prob, step_index, base_seed(seed), m, ctx->stream), "mask");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

static npa_status check_decode(npa_context* ctx, uint32_t S, const npa_gaussian_decode_cfg* cfg) {
    if (!cfg) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null decode config");
    const uint32_t K = cfg->mode == NPA_DECODE_SH0_ORIENTED ? (cfg->sh_degree + 1) * (cfg->sh_degree + 1) : 1;
    switch (cfg->mode) {  // validate_decode_layout gaussian.rs:102-125
        case NPA_DECODE_PARTICLE_POINT:
        case NPA_DECODE_SH0_FIXED_SCALE:
            if (S < 3) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "state_dims must include an RGB tail for SH0 gaussian decoding");
            break;
        case NPA_DECODE_SH0_LEARNED_SCALE:
            if (S < 5) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "state_dims must include scale, opacity, and RGB tail channels");
            break;
        case NPA_DECODE_SH0_ORIENTED:
            if (cfg->sh_degree > 8 || S < K * 3 + 8)
                return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                            "state_dims must fit color/sh, rotation, and anisotropy/opacity tails");
            break;
        default:
            return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: unknown decode mode");
    }
    return NPA_OK;
}

npa_status npa_decode_gaussians_3d(npa_context* ctx, const float* positions, const float* states, uint32_t count,
                                   uint32_t S, const npa_gaussian_decode_cfg* cfg, float* pv, float* sh, float* rot,
                                   float* so) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_decode(ctx, S, cfg);
    if (st) return st;
    if (count && (st = need(ctx, {positions, states, pv, sh, rot, so}, "input or output array"))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint32_t K = cfg->mode == NPA_DECODE_SH0_ORIENTED ? (cfg->sh_degree + 1) * (cfg->sh_degree + 1) : 1;
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, (uint64_t)count * 16);
    const float* s = io.in(states, (uint64_t)count * S * 4);
    float* dpv = io.out(pv, (uint64_t)count * 16);
    float* dsh = io.out(sh, (uint64_t)count * K * 12);
    float* drot = io.out(rot, (uint64_t)count * 16);
    float* dso = io.out(so, (uint64_t)count * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (count && (!aligned16(pos) || !aligned16(dpv) || !aligned16(drot) || !aligned16(dso)))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: 4-wide arrays must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_decode_gaussians(pos, s, count, S, *cfg, dpv, dsh, drot, dso, ctx->stream), "decode");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

static npa_status check_splat(npa_context* ctx, const npa_splat2d_cfg* cfg) {
    if (!cfg) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null splat config");
    if (cfg->image_size == 0 || cfg->image_size > 4096)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: splat image_size must be in 1..=4096");
    float sigma = cfg->sigma;
    if (cfg->normalize_color) sigma = sigma * (float)cfg->image_size * cfg->pixel_size / (cfg->hi - cfg->lo);
    const float r = ceilf(5.0f * sigma);
    if (!(r <= 1024.0f))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: splat radius ceil(5*sigma) must be <= 1024 pixels");
    return NPA_OK;
}

npa_status npa_splat_2d(npa_context* ctx, const float* positions, const float* colors, uint32_t count,
                        const npa_splat2d_cfg* cfg, float* image) {
    if (!ctx || !image) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_splat(ctx, cfg);
    if (st) return st;
    if (count && (!colors || !positions)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null positions or colors");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, (uint64_t)count * 16);
    const float* col = io.in(colors, (uint64_t)count * 12);
    float* img = io.out(image, (uint64_t)cfg->image_size * cfg->image_size * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if ((count && !aligned16(pos)) || !aligned16(img))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions and image must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_splat_2d(pos, col, nullptr, 3, count, *cfg, img, ctx->splat_ws, ctx->stream, &ctx->prof,
                                      count ? count : 1u, 1u, 1u),
            "splat");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

// Window grid of a tiled splat: rows of tiles_x windows, each image_size pixels square.
static npa_status check_tiling(npa_context* ctx, const npa_splat2d_cfg* cfg, uint32_t B, uint32_t N, uint32_t tiles_x,
                               uint64_t* pixels) {
    if (B == 0 || N == 0) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: empty batch");
    if (tiles_x == 0 || tiles_x > B)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: tiles_x must be in 1..=batch_size");
    const uint64_t rows = (B + tiles_x - 1) / tiles_x;
    const uint64_t side = cfg->image_size;
    const uint64_t tiles_per_win = ((side + 15) / 16) * ((side + 15) / 16);
    if (rows * tiles_x * tiles_per_win > 65536 || tiles_x * side > 16384 || rows * side > 16384)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: tiled image too large (at most 65536 16x16 tiles, 16384 pixels a side)");
    if ((uint64_t)B * N >= (1ull << 31)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many particles");
    *pixels = rows * side * tiles_x * side;
    return NPA_OK;
}

npa_status npa_splat_2d_tiled(npa_context* ctx, const float* positions, const float* colors, uint32_t B, uint32_t N,
                              const npa_splat2d_cfg* cfg, uint32_t tiles_x, float* image) {
    if (!ctx || !image) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_splat(ctx, cfg);
    if (st) return st;
    uint64_t pixels = 0;
    if ((st = check_tiling(ctx, cfg, B, N, tiles_x, &pixels))) return st;
    if (!colors || !positions) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null positions or colors");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint32_t count = B * N;
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, (uint64_t)count * 16);
    const float* col = io.in(colors, (uint64_t)count * 12);
    float* img = io.out(image, pixels * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(pos) || !aligned16(img))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions and image must be 16-byte aligned");
    const uint32_t windows = (B + tiles_x - 1) / tiles_x * tiles_x;
    NPA_HIP(ctx, npa::launch_splat_2d(pos, col, nullptr, 3, count, *cfg, img, ctx->splat_ws, ctx->stream, &ctx->prof, N,
                                      windows, tiles_x),
            "splat");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

// validate_render_loss_config (render_loss/attributes.rs:114-174), then this library's limits.
static npa_status check_render(npa_context* ctx, const npa_render_cfg* cfg, const uint32_t* views, uint32_t nviews) {
    if (!cfg) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null render config");
    auto bad = [&](const std::string& m) { return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + m); };
    if (cfg->image_size == 0) return bad("render loss image_size must be non-zero");
    if (cfg->target_samples == 0) return bad("render loss target_samples must be non-zero");
    if (!std::isfinite(cfg->sigma) || cfg->sigma <= 0.0f)
        return bad("render loss sigma must be finite and positive, got " + fmt_f(cfg->sigma));
    if (!std::isfinite(cfg->min_sigma) || cfg->min_sigma <= 0.0f)
        return bad("render loss min_sigma must be finite and positive, got " + fmt_f(cfg->min_sigma));
    if (!std::isfinite(cfg->max_sigma) || cfg->max_sigma < cfg->min_sigma)
        return bad("render loss max_sigma must be finite and >= min_sigma, got max=" + fmt_f(cfg->max_sigma) +
                   " min=" + fmt_f(cfg->min_sigma));
    if (!std::isfinite(cfg->world_scale) || cfg->world_scale <= 0.0f)
        return bad("render loss world_scale must be finite and positive, got " + fmt_f(cfg->world_scale));
    if (!std::isfinite(cfg->opacity_logit_bias))
        return bad("render loss opacity_logit_bias must be finite, got " + fmt_f(cfg->opacity_logit_bias));
    if (!std::isfinite(cfg->density_weight) || cfg->density_weight < 0.0f)
        return bad("render loss density_weight must be finite and non-negative, got " + fmt_f(cfg->density_weight));
    if (!std::isfinite(cfg->color_weight) || cfg->color_weight < 0.0f)
        return bad("render loss color_weight must be finite and non-negative, got " + fmt_f(cfg->color_weight));
    if (!std::isfinite(cfg->depth_weight) || cfg->depth_weight < 0.0f)
        return bad("render loss depth_weight must be finite and non-negative, got " + fmt_f(cfg->depth_weight));
    if (cfg->gaussian_decode_mode > NPA_DECODE_SH0_ORIENTED) return bad("unknown gaussian decode mode");
    if (cfg->image_size > 4096) return bad("render image_size must be <= 4096");
    if (!(ceilf(5.0f * cfg->max_sigma) <= 1024.0f)) return bad("render radius ceil(5*max_sigma) must be <= 1024 pixels");
    if (nviews == 0 || nviews > npa::kMaxRenderViews || !views) return bad("render needs 1..=16 views");
    for (uint32_t v = 0; v < nviews; ++v)
        if (views[v] > NPA_VIEW_ISO) return bad("unknown render view " + std::to_string(views[v]));
    const uint64_t t = (cfg->image_size + 15) / 16;
    if (t * t * nviews > 65536) return bad("render images too large (at most 65536 16x16 tiles over all views)");
    return NPA_OK;
}

npa_status npa_render_views(npa_context* ctx, const float* positions, const float* colors, const float* opacities,
                            const float* sigmas, uint32_t count, const uint32_t* views, uint32_t nviews,
                            const npa_render_cfg* cfg, float* images) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_render(ctx, cfg, views, nviews);
    if (st) return st;
    if (!images) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null images");
    if (count && (!positions || !colors || !opacities || !sigmas))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null particle arrays");
    if ((uint64_t)count * nviews >= (1ull << 31))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many particles");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t px = (uint64_t)cfg->image_size * cfg->image_size * nviews;
    HostIO io(ctx);
    const float4* pos = (const float4*)io.in(positions, (uint64_t)count * 16);
    const float* col = io.in(colors, (uint64_t)count * 12);
    const float* op = io.in(opacities, (uint64_t)count * 4);
    const float* sg = io.in(sigmas, (uint64_t)count * 4);
    float* img = io.out(images, px * 20);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (count && !aligned16(pos)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: positions must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_render_views(pos, col, op, sg, count, views, nviews, *cfg, img, ctx->splat_ws, ctx->stream,
                                          &ctx->prof),
            "render");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

static npa_status check_render_states(npa_context* ctx, uint32_t S, const npa_render_cfg* cfg) {
    if (S < 3)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: render loss needs at least 3 state channels for color, got " + std::to_string(S));
    if (cfg->gaussian_decode_mode == NPA_DECODE_SH0_LEARNED_SCALE && S < 5)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: learned-scale render decode needs at least 5 state channels, got " +
                        std::to_string(S));
    return NPA_OK;
}

npa_status npa_render_attributes(npa_context* ctx, const float* states, uint32_t count, uint32_t S,
                                 const npa_render_cfg* cfg, float* colors, float* opacities, float* sigmas,
                                 float* derivatives) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    if (!cfg) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null render config");
    npa_status st = check_render_states(ctx, S, cfg);
    if (st) return st;
    if (cfg->gaussian_decode_mode > NPA_DECODE_SH0_ORIENTED)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: unknown gaussian decode mode");
    if (count && (!states || !colors || !opacities || !sigmas))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null attribute arrays");
    if ((uint64_t)count * S >= (1ull << 40)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many particles");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    const float* s = io.in(states, (uint64_t)count * S * 4);
    float* col = io.out(colors, (uint64_t)count * 12);
    float* op = io.out(opacities, (uint64_t)count * 4);
    float* sg = io.out(sigmas, (uint64_t)count * 4);
    float* dv = derivatives ? io.out(derivatives, (uint64_t)count * 4) : nullptr;
    if (io.err) return hip_fail(ctx, io.err, "staging");
    NPA_HIP(ctx, npa::launch_render_attributes(s, count, S, *cfg, col, op, sg, dv, ctx->stream), "render attributes");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

// ==================================================================== executor
npa_status npa_state_create(npa_context* ctx, const npa_model_cfg* model, const npa_weights* w,
                            const npa_grid_cfg* grid, const float* positions, const float* states, uint32_t B,
                            uint32_t N, float dt, float update_prob, uint64_t seed, npa_state** out) {
    if (!ctx || !w || !out) return NPA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    npa_status st = validate_grid(ctx, grid);
    if (st) return st;
    if ((st = check_model(ctx, model, grid))) return st;
    const uint64_t total = (uint64_t)B * N;
    if (total == 0) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: empty particle system");
    if ((st = need(ctx, {positions, states}, "positions or states"))) return st;
    if ((st = need_weights(ctx, w, model_perception_dims(*model), model->hidden_dims,
                           model->spatial_dims + model->state_dims)))
        return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    npa::HashgridPlan plan;
    std::string err;
    if (!npa::make_plan(*grid, B, N, &plan, &err))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + err);
    npa_state* s = new npa_state();
    s->ctx = ctx;
    s->model = *model;
    s->grid = *grid;
    s->B = B;
    s->N = N;
    s->dt = dt;
    s->update_prob = update_prob;
    s->seed = seed;
    s->plan = plan;
    s->grid_blocks = grid_blocks_for(ctx, plan);
    const uint32_t S = model->state_dims, F = model_perception_dims(*model), H = model->hidden_dims;
    const uint32_t O = model->spatial_dims + S;
    const hipMemcpyKind kind = ctx->host_io ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    hipError_t e = hipSuccess;
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
        e = s->pos[k].reserve(total * 16);
        if (e == hipSuccess) e = s->states[k].reserve(total * S * 4);
    }
    if (e == hipSuccess) e = s->density.reserve(total * 4);
    if (e == hipSuccess) e = s->w1.reserve((uint64_t)H * F * 4 + 4);
    if (e == hipSuccess) e = s->b1.reserve((uint64_t)H * 4 + 4);
    if (e == hipSuccess) e = s->w2.reserve((uint64_t)O * H * 4 + 4);
    if (e == hipSuccess) e = s->b2.reserve((uint64_t)O * 4 + 4);
    const npa::StepParams sp = [&] {
        npa::StepParams q = make_params(*grid, opts_for_model(*model), B, N, S);
        apply_model(&q, *model, grid->eps);
        return q;
    }();
    if (e == hipSuccess) e = s->ws.reserve(plan, total, B, S, (int)grid->dim, feature_rows_for(sp));
    if (e == hipSuccess) e = s->ws.wpad.reserve(npa::padded_weight_floats(sp) * 4);
    if (e == hipSuccess) e = hipMemcpyAsync(s->pos[0].ptr, positions, total * 16, kind, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(s->states[0].ptr, states, total * S * 4, kind, ctx->stream);
    if (e == hipSuccess && (uint64_t)H * F) e = hipMemcpyAsync(s->w1.ptr, w->w1, (uint64_t)H * F * 4, kind, ctx->stream);
    if (e == hipSuccess && H) e = hipMemcpyAsync(s->b1.ptr, w->b1, (uint64_t)H * 4, kind, ctx->stream);
    if (e == hipSuccess && (uint64_t)O * H) e = hipMemcpyAsync(s->w2.ptr, w->w2, (uint64_t)O * H * 4, kind, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(s->b2.ptr, w->b2, (uint64_t)O * 4, kind, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(s->density.ptr, 0, total * 4, ctx->stream);
    if (e == hipSuccess)
        e = npa::launch_pad_weights(sp, s->w1.as<float>(), s->b1.as<float>(), s->w2.as<float>(), s->b2.as<float>(),
                                    s->ws.wpad.as<float>(), ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        delete s;
        return hip_fail(ctx, e, "state create");
    }
    ctx->refs.fetch_add(1);
    *out = s;
    return NPA_OK;
}

void npa_state_destroy(npa_state* s) {
    if (!s) return;
    npa_context* ctx = s->ctx;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    delete s;
    context_release(ctx);
}

npa_status npa_state_step(npa_state* s, uint32_t steps) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint32_t S = s->model.state_dims;
    npa::StepParams p = make_params(s->grid, opts_for_model(s->model), s->B, s->N, S);
    apply_model(&p, s->model, s->grid.eps);
    p.dt = s->dt;
    p.update_prob = s->update_prob;
    p.base_seed = base_seed(s->seed);
    p.mlp_engine = (uint32_t)s->mlp_engine;
    npa::StepIO io;
    io.w1 = s->w1.as<float>();
    io.b1 = s->b1.as<float>();
    io.w2 = s->w2.as<float>();
    io.b2 = s->b2.as<float>();
    for (uint32_t k = 0; k < steps; ++k) {
        const int c = s->cur;
        p.step_index = (uint32_t)s->step_index;
        io.pos = s->pos[c].as<float4>();
        io.states = s->states[c].as<float>();
        io.out_pos = s->pos[1 - c].as<float4>();
        io.out_states = s->states[1 - c].as<float>();
        const npa::SplitTargets targets = npa::step_targets(p, io);
        NPA_HIP(ctx, npa::launch_hashgrid(s->plan, p.g, io.pos, io.states, S, s->B, s->N, s->ws, true, ctx->stream,
                                          &ctx->prof, &targets),
                "hashgrid");
        NPA_HIP(ctx, npa::launch_density(p, s->ws, s->density.as<float>(), s->grid_blocks, ctx->stream, &ctx->prof),
                "density");
        NPA_HIP(ctx, npa::launch_update(p, s->ws, io, 0, s->grid_blocks, ctx->stream, &ctx->prof), "update");
        s->cur = 1 - c;
        s->step_index += 1;
    }
    return NPA_OK;
}

npa_status npa_state_set_mlp_engine(npa_state* s, int engine) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    if (engine != NPA_MLP_VALU && engine != NPA_MLP_MFMA && engine != NPA_MLP_MFMA_BF16)
        return fail(s->ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: unknown MLP engine " + std::to_string(engine));
    s->mlp_engine = engine;
    return NPA_OK;
}

npa_status npa_state_read(npa_state* s, float* positions, float* states, float* density) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t total = (uint64_t)s->B * s->N;
    const hipMemcpyKind kind = ctx->host_io ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    if (positions) NPA_HIP(ctx, hipMemcpyAsync(positions, s->pos[s->cur].ptr, total * 16, kind, ctx->stream), "read pos");
    if (states)
        NPA_HIP(ctx, hipMemcpyAsync(states, s->states[s->cur].ptr, total * s->model.state_dims * 4, kind, ctx->stream),
                "read states");
    if (density) NPA_HIP(ctx, hipMemcpyAsync(density, s->density.ptr, total * 4, kind, ctx->stream), "read density");
    return check_flags(ctx, s->ws);
}

npa_status npa_state_update_model(npa_state* s, const npa_weights* w) {
    if (!s || !w) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    const npa_model_cfg& m = s->model;
    const uint32_t F = model_perception_dims(m), H = m.hidden_dims, O = m.spatial_dims + m.state_dims;
    npa_status st = need_weights(ctx, w, F, H, O);
    if (st) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const hipMemcpyKind kind = ctx->host_io ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    if ((uint64_t)H * F) NPA_HIP(ctx, hipMemcpyAsync(s->w1.ptr, w->w1, (uint64_t)H * F * 4, kind, ctx->stream), "w1");
    if (H) NPA_HIP(ctx, hipMemcpyAsync(s->b1.ptr, w->b1, (uint64_t)H * 4, kind, ctx->stream), "b1");
    if ((uint64_t)O * H) NPA_HIP(ctx, hipMemcpyAsync(s->w2.ptr, w->w2, (uint64_t)O * H * 4, kind, ctx->stream), "w2");
    NPA_HIP(ctx, hipMemcpyAsync(s->b2.ptr, w->b2, (uint64_t)O * 4, kind, ctx->stream), "b2");
    npa::StepParams sp = make_params(s->grid, opts_for_model(m), s->B, s->N, m.state_dims);
    apply_model(&sp, m, s->grid.eps);
    NPA_HIP(ctx, npa::launch_pad_weights(sp, s->w1.as<float>(), s->b1.as<float>(), s->w2.as<float>(),
                                         s->b2.as<float>(), s->ws.wpad.as<float>(), ctx->stream),
            "pad weights");
    if (ctx->host_io) NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "sync");
    return NPA_OK;
}

npa_status npa_state_step_index(const npa_state* s, uint64_t* step_index) {
    if (!s || !step_index) return NPA_ERR_INVALID_ARGUMENT;
    *step_index = s->step_index;
    return NPA_OK;
}

npa_status npa_state_buffers(npa_state* s, float** positions, float** states) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    if (positions) *positions = s->pos[s->cur].as<float>();
    if (states) *states = s->states[s->cur].as<float>();
    return NPA_OK;
}

npa_status npa_state_splat_2d(npa_state* s, const npa_splat2d_cfg* cfg, float* image) {
    if (!s || !image) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = check_splat(ctx, cfg);
    if (st) return st;
    if (s->model.state_dims < 3)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: splat colours need state_dims >= 3");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t total = (uint64_t)s->B * s->N;
    if (total >= (1ull << 32)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many particles");
    HostIO io(ctx);
    float* img = io.out(image, (uint64_t)cfg->image_size * cfg->image_size * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(img)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: image must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_splat_2d(s->pos[s->cur].as<float4>(), nullptr, s->states[s->cur].as<float>(),
                                      s->model.state_dims, (uint32_t)total, *cfg, img, s->splat_ws, ctx->stream,
                                      &ctx->prof, (uint32_t)total, 1u, 1u),
            "splat");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_state_splat_2d_tiled(npa_state* s, const npa_splat2d_cfg* cfg, uint32_t tiles_x, float* image) {
    if (!s || !image) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = check_splat(ctx, cfg);
    if (st) return st;
    if (s->model.state_dims < 3)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: splat colours need state_dims >= 3");
    uint64_t pixels = 0;
    if ((st = check_tiling(ctx, cfg, s->B, s->N, tiles_x, &pixels))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    HostIO io(ctx);
    float* img = io.out(image, pixels * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(img)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: image must be 16-byte aligned");
    const uint32_t windows = (s->B + tiles_x - 1) / tiles_x * tiles_x;
    NPA_HIP(ctx, npa::launch_splat_2d(s->pos[s->cur].as<float4>(), nullptr, s->states[s->cur].as<float>(),
                                      s->model.state_dims, s->B * s->N, *cfg, img, s->splat_ws, ctx->stream,
                                      &ctx->prof, s->N, windows, tiles_x),
            "splat");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_state_render_views(npa_state* s, const uint32_t* views, uint32_t nviews, const npa_render_cfg* cfg,
                                  float* images) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = check_render(ctx, cfg, views, nviews);
    if (st) return st;
    if (!images) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null images");
    const uint32_t S = s->model.state_dims;
    if ((st = check_render_states(ctx, S, cfg))) return st;
    if (s->B != 1)  // validate_render_trace (attributes.rs:89-112)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: render loss expects batch_size=1, got " + std::to_string(s->B));
    const uint32_t n = s->N;
    if ((uint64_t)n * nviews >= (1ull << 31)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many particles");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    NPA_HIP(ctx, s->splat_ws.attrs.reserve((uint64_t)(n ? n : 1) * 20), "render attributes");
    float* col = s->splat_ws.attrs.as<float>();
    float* op = col + 3 * (uint64_t)n;
    float* sg = op + n;
    HostIO io(ctx);
    float* img = io.out(images, (uint64_t)cfg->image_size * cfg->image_size * nviews * 20);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    NPA_HIP(ctx, npa::launch_render_attributes(s->states[s->cur].as<float>(), n, S, *cfg, col, op, sg, nullptr,
                                               ctx->stream),
            "render attributes");
    NPA_HIP(ctx, npa::launch_render_views(s->pos[s->cur].as<float4>(), col, op, sg, n, views, nviews, *cfg, img,
                                          s->splat_ws, ctx->stream, &ctx->prof),
            "render");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_state_decode_gaussians_3d(npa_state* s, const npa_gaussian_decode_cfg* cfg, float* pv, float* sh,
                                         float* rot, float* so) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    const uint32_t S = s->model.state_dims;
    npa_status st = check_decode(ctx, S, cfg);
    if (st) return st;
    if ((st = need(ctx, {pv, sh, rot, so}, "output array"))) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t total = (uint64_t)s->B * s->N;
    const uint32_t K = cfg->mode == NPA_DECODE_SH0_ORIENTED ? (cfg->sh_degree + 1) * (cfg->sh_degree + 1) : 1;
    HostIO io(ctx);
    float* dpv = io.out(pv, total * 16);
    float* dsh = io.out(sh, total * K * 12);
    float* drot = io.out(rot, total * 16);
    float* dso = io.out(so, total * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(dpv) || !aligned16(drot) || !aligned16(dso))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: 4-wide arrays must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_decode_gaussians(s->pos[s->cur].as<float4>(), s->states[s->cur].as<float>(),
                                              (uint32_t)total, S, *cfg, dpv, dsh, drot, dso, ctx->stream),
            "decode");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

static npa_status check_raster_camera(npa_context* ctx, const npa_raster_camera* cam) {
    if (!cam) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null raster camera");
    auto bad = [&](const std::string& m) { return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: " + m); };
    if (cam->width == 0 || cam->height == 0) return bad("raster width and height must be non-zero");
    if (cam->width > 16384 || cam->height > 16384) return bad("raster width and height must be <= 16384");
    const uint64_t tiles = (uint64_t)((cam->width + 15) / 16) * ((cam->height + 15) / 16);
    if (tiles > 65536) return bad("raster image too large (at most 65536 16x16 tiles)");
    if (cam->sh_degree > 3) return bad("raster sh_degree must be <= 3, got " + std::to_string(cam->sh_degree));
    if (cam->color_mode > NPA_RASTER_COLOR_RGB) return bad("unknown raster color mode");
    for (int k = 0; k < 16; ++k)
        if (!std::isfinite(cam->view[k])) return bad("raster view matrix must be finite");
    if (!std::isfinite(cam->fx) || cam->fx <= 0.0f || !std::isfinite(cam->fy) || cam->fy <= 0.0f)
        return bad("raster focal lengths must be finite and positive");
    if (!std::isfinite(cam->cx) || !std::isfinite(cam->cy)) return bad("raster principal point must be finite");
    if (!std::isfinite(cam->near_plane) || cam->near_plane <= 0.0f)
        return bad("raster near_plane must be finite and positive, got " + fmt_f(cam->near_plane));
    if (!(cam->far_plane > cam->near_plane))
        return bad("raster far_plane must exceed near_plane, got " + fmt_f(cam->far_plane));
    return NPA_OK;
}

npa_status npa_raster_gaussians_3d(npa_context* ctx, const float* position_visibility, const float* spherical_harmonic,
                                   const float* rotation, const float* scale_opacity, uint32_t count,
                                   const npa_raster_camera* camera, float* image) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    npa_status st = check_raster_camera(ctx, camera);
    if (st) return st;
    if (!image) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null image");
    if (count && (!position_visibility || !spherical_harmonic || !rotation || !scale_opacity))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null Gaussian arrays");
    if (count >= (1u << 31)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many Gaussians");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t K = (uint64_t)(camera->sh_degree + 1) * (camera->sh_degree + 1);
    HostIO io(ctx);
    const float4* pv = (const float4*)io.in(position_visibility, (uint64_t)count * 16);
    const float* sh = io.in(spherical_harmonic, (uint64_t)count * K * 12);
    const float4* rot = (const float4*)io.in(rotation, (uint64_t)count * 16);
    const float4* so = (const float4*)io.in(scale_opacity, (uint64_t)count * 16);
    float* img = io.out(image, (uint64_t)camera->width * camera->height * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if ((count && (!aligned16(pv) || !aligned16(rot) || !aligned16(so))) || !aligned16(img))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: 4-wide arrays and the image must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_raster_gaussians(pv, sh, rot, so, count, *camera, img, ctx->splat_ws, ctx->stream,
                                              &ctx->prof),
            "raster");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

// Gaussian buffers of a state's export: `count` entries of each array, at least B*N
// (write_state_into_gaussian_bind_group_impl steps.rs:93-98).
static npa_status check_export(npa_context* ctx, const npa_state* s, uint32_t count, std::initializer_list<const void*> arrays) {
    const uint64_t total = (uint64_t)s->B * s->N;
    if (count < total)
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT,
                    "invalid argument: gaussian bind group count " + std::to_string(count) +
                        " is smaller than automata particle count " + std::to_string(total));
    return need(ctx, arrays, "Gaussian array");
}

// The export of the state's current buffers into device (or staged host) arrays.
static npa_status write_export(npa_state* s, float* pv, float* sh, float* rot, float* so) {
    npa_context* ctx = s->ctx;
    const uint64_t total = (uint64_t)s->B * s->N;
    HostIO io(ctx);
    float* dpv = io.out(pv, total * 16);
    float* dsh = io.out(sh, total * NPA_GAUSSIAN_SH_COEFF_COUNT * 4);
    float* drot = io.out(rot, total * 16);
    float* dso = io.out(so, total * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(dpv) || !aligned16(dsh) || !aligned16(drot) || !aligned16(dso))
        return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: Gaussian arrays must be 16-byte aligned");
    NPA_HIP(ctx, npa::launch_write_gaussians(s->pos[s->cur].as<float4>(), s->states[s->cur].as<float>(),
                                             (uint32_t)total, s->N, s->model.state_dims, s->model.spatial_dims,
                                             s->grid.eps, s->model.position_features != 0, dpv, dsh, drot, dso,
                                             ctx->stream),
            "gaussian export");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_state_write_gaussians(npa_state* s, uint32_t count, float* pv, float* sh, float* rot, float* so) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = check_export(ctx, s, count, {pv, sh, rot, so});
    if (st) return st;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    return write_export(s, pv, sh, rot, so);
}

npa_status npa_state_step_into_gaussians(npa_state* s, uint32_t steps, uint32_t count, float* pv, float* sh,
                                         float* rot, float* so) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = check_export(ctx, s, count, {pv, sh, rot, so});
    if (st) return st;
    if ((st = npa_state_step(s, steps ? steps : 1u))) return st;
    return write_export(s, pv, sh, rot, so);
}

npa_status npa_state_raster_gaussians_3d(npa_state* s, const npa_gaussian_decode_cfg* cfg,
                                         const npa_raster_camera* camera, float* image) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    npa_status st = NPA_OK;
    if (cfg && (st = check_decode(ctx, s->model.state_dims, cfg))) return st;
    st = check_raster_camera(ctx, camera);
    if (st) return st;
    if (!image) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: null image");
    npa_raster_camera cam = *camera;
    // the export carries SH coefficients (degree-3 layout, DC only); the decode carries colours in
    // the first of its K coefficient triples per Gaussian (K = (sh_degree + 1)^2 in oriented mode),
    // so the raster reads them at that stride
    cam.sh_degree = cfg ? 0u : 3u;
    cam.color_mode = cfg ? NPA_RASTER_COLOR_RGB : NPA_RASTER_COLOR_SH;
    const uint32_t K = cfg ? (cfg->mode == NPA_DECODE_SH0_ORIENTED ? (cfg->sh_degree + 1) * (cfg->sh_degree + 1) : 1u)
                           : NPA_GAUSSIAN_SH_COEFF_COUNT / 3;
    const uint64_t total = (uint64_t)s->B * s->N;
    if (total >= (1ull << 31)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: too many Gaussians");
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint64_t t1 = total ? total : 1;
    const uint64_t sh_bytes = (t1 * K * 12 + 15) / 16 * 16;
    NPA_HIP(ctx, ctx->splat_ws.decoded.reserve(t1 * 48 + sh_bytes), "alloc");
    char* base = ctx->splat_ws.decoded.as<char>();
    float* dpv = (float*)base;
    float* drot = (float*)(base + t1 * 16);
    float* dso = (float*)(base + t1 * 32);
    float* dsh = (float*)(base + t1 * 48);
    HostIO io(ctx);
    float* img = io.out(image, (uint64_t)cam.width * cam.height * 16);
    if (io.err) return hip_fail(ctx, io.err, "staging");
    if (!aligned16(img)) return fail(ctx, NPA_ERR_INVALID_ARGUMENT, "invalid argument: the image must be 16-byte aligned");
    if (cfg)
        NPA_HIP(ctx, npa::launch_decode_gaussians(s->pos[s->cur].as<float4>(), s->states[s->cur].as<float>(),
                                                  (uint32_t)total, s->model.state_dims, *cfg, dpv, dsh, drot, dso,
                                                  ctx->stream),
                "decode");
    else
        NPA_HIP(ctx, npa::launch_write_gaussians(s->pos[s->cur].as<float4>(), s->states[s->cur].as<float>(),
                                                 (uint32_t)total, s->N, s->model.state_dims, s->model.spatial_dims,
                                                 s->grid.eps, s->model.position_features != 0, dpv, dsh, drot, dso,
                                                 ctx->stream),
                "gaussian export");
    NPA_HIP(ctx, npa::launch_raster_gaussians((const float4*)dpv, dsh, (const float4*)drot, (const float4*)dso,
                                              (uint32_t)total, cam, img, ctx->splat_ws, ctx->stream, &ctx->prof, K),
            "raster");
    NPA_HIP(ctx, io.finish(), "host io");
    return NPA_OK;
}

npa_status npa_state_pair_counts(npa_state* s, uint64_t* candidates, uint64_t* pairs, uint64_t* targets,
                                 uint64_t* target_candidates, uint64_t* target_pairs) {
    if (!s) return NPA_ERR_INVALID_ARGUMENT;
    npa_context* ctx = s->ctx;
    if (set_device(ctx)) return NPA_ERR_DEVICE;
    const uint32_t S = s->model.state_dims;
    npa::StepParams p = make_params(s->grid, opts_for_model(s->model), s->B, s->N, S);
    p.g.spatial = 0;  // the reference's bins: candidates count every particle of a neighbour cell's bin
    p.update_prob = s->update_prob;
    p.base_seed = base_seed(s->seed);
    p.step_index = (uint32_t)s->step_index;
    NPA_HIP(ctx, npa::launch_hashgrid(s->plan, p.g, s->pos[s->cur].as<float4>(), s->states[s->cur].as<float>(), S,
                                      s->B, s->N, s->ws, true, ctx->stream, nullptr),
            "hashgrid");
    NPA_HIP(ctx, hipMemsetAsync(s->ws.counters.ptr, 0, 40, ctx->stream), "zero counters");
    NPA_HIP(ctx, npa::launch_count_pairs(p, s->ws, s->grid_blocks, s->ws.counters.as<unsigned long long>(), ctx->stream),
            "count");
    unsigned long long h[5] = {0, 0, 0, 0, 0};
    NPA_HIP(ctx, hipMemcpyAsync(h, s->ws.counters.ptr, 40, hipMemcpyDeviceToHost, ctx->stream), "readback");
    NPA_HIP(ctx, hipStreamSynchronize(ctx->stream), "sync");
    if (candidates) *candidates = h[0];
    if (pairs) *pairs = h[1];
    if (targets) *targets = h[2];
    if (target_candidates) *target_candidates = h[3];
    if (target_pairs) *target_pairs = h[4];
    return check_flags(ctx, s->ws);
}

// ================================================================== profiling
npa_status npa_profile_enable(npa_context* ctx, int kernel_mask) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    ctx->prof.enabled = kernel_mask != 0;
    ctx->prof.mask = (uint32_t)kernel_mask;
    return NPA_OK;
}

npa_status npa_profile_reset(npa_context* ctx) {
    if (!ctx) return NPA_ERR_INVALID_ARGUMENT;
    NPA_HIP(ctx, ctx->prof.collect(), "profile collect");
    ctx->prof.reset();
    return NPA_OK;
}

npa_status npa_profile_read(npa_context* ctx, int kernel_id, double* total_ms, uint64_t* launches) {
    if (!ctx || kernel_id < 0 || kernel_id >= NPA_KERNEL_COUNT) return NPA_ERR_INVALID_ARGUMENT;
    NPA_HIP(ctx, ctx->prof.collect(), "profile collect");
    if (total_ms) *total_ms = ctx->prof.total_ms[kernel_id];
    if (launches) *launches = ctx->prof.launches[kernel_id];
    return NPA_OK;
}

}  // extern "C"

// ============================================================ profiler impl
namespace npa {

hipEvent_t Profiler::get() {
    if (!pool.empty()) {
        hipEvent_t e = pool.back();
        pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

bool Profiler::pick(int kernel, hipEvent_t* a, hipEvent_t* b) {
    *a = get();
    if (!*a) return false;
    *b = get();
    if (!*b) {
        pool.push_back(*a);
        return false;
    }
    pending.push_back({*a, *b, kernel});
    return true;
}

void Profiler::begin(int kernel, hipStream_t s, hipEvent_t* ev) {
    (void)kernel;
    *ev = get();
    if (*ev) (void)hipEventRecord(*ev, s);
}

void Profiler::end(int kernel, hipStream_t s, hipEvent_t a) {
    hipEvent_t b = get();
    if (!b) return;
    (void)hipEventRecord(b, s);
    pending.push_back({a, b, kernel});
}

hipError_t Profiler::collect() {
    for (const Pair& p : pending) {
        hipError_t e = hipEventSynchronize(p.b);
        if (e != hipSuccess) return e;
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, p.a, p.b);
        if (e != hipSuccess) return e;
        total_ms[p.kernel] += ms;
        launches[p.kernel] += 1;
        pool.push_back(p.a);
        pool.push_back(p.b);
    }
    pending.clear();
    return hipSuccess;
}

void Profiler::reset() {
    for (int k = 0; k < NPA_KERNEL_COUNT; ++k) {
        total_ms[k] = 0.0;
        launches[k] = 0;
    }
}

Profiler::~Profiler() {
    for (const Pair& p : pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
}

}  // namespace npa
