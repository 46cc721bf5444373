/*
 * npa_abi.h - C ABI of the MI355X-native fixed-NPA rollout library (libnpa_hip.so).
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, and is
 * stream-ordered on the stream owned by (or handed to) its npa_context.
 * Array arguments are DEVICE pointers unless the context was switched to host
 * I/O with npa_context_set_host_io(ctx, 1); then they are host pointers, the
 * library stages them through device buffers it owns and the call returns
 * only after the results are back in host memory.
 *
 * Layouts follow the reference (burn_automata_kernels, Rust):
 *   positions  [B*N][4]   f32  (x, y, z, w)          `&[[f32; 4]]`
 *   states     [B*N][S]   f32  row-major             `&[f32]`
 *   features   [B*N][F]   f32  [state | blur | grad(S*d, channel-major) | dgrad(d)? | pos(d)?]
 *   weights    w1[H][F], b1[H], w2[O][H], b2[O], O = d + S
 * Index tables use u32 where the reference uses usize; sizes must keep
 * B*N and B*C below 2^32 (checked, NPA_ERR_INVALID_ARGUMENT otherwise).
 *
 * Status codes map 1:1 onto `KernelError` variants
 * (crates/burn_automata_kernels/src/config.rs:101-137); npa_last_error()
 * returns the formatted message of the last failing call on a context.
 */
#ifndef NPA_ABI_H
#define NPA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
typedef enum npa_status {
    NPA_OK = 0,
    NPA_ERR_INVALID_DIM = 1,           /* KernelError::InvalidDim */
    NPA_ERR_INVALID_EPS = 2,           /* KernelError::InvalidEps */
    NPA_ERR_INVALID_GRID_SIZE = 3,     /* KernelError::InvalidGridSize */
    NPA_ERR_PARTICLE_MODE_POW2 = 4,    /* KernelError::ParticleModeRequiresPowerOfTwo */
    NPA_ERR_POSITION_SHAPE = 10,       /* KernelError::PositionShape */
    NPA_ERR_STATE_SHAPE = 11,          /* KernelError::StateShape */
    NPA_ERR_OUTPUT_SHAPE = 12,         /* KernelError::OutputShape */
    NPA_ERR_INVALID_ARGUMENT = 13,     /* KernelError::InvalidArgument */
    NPA_ERR_INVALID_MODEL = 20,        /* AutomataError::InvalidModel (crates/burn_automata/src/error.rs) */
    NPA_ERR_IO = 21,                   /* AutomataError::Io */
    NPA_ERR_JSON = 22,                 /* AutomataError::Json */
    NPA_ERR_INVALID_FORMAT = 23,       /* AutomataError::InvalidFormat */
    NPA_ERR_DEVICE = 30,               /* HIP runtime failure */
    NPA_ERR_OUT_OF_MEMORY = 31,
    NPA_ERR_COORD_OVERFLOW = 32        /* a Particle-mode cell coordinate left +-2^30 (see below) */
} npa_status;

/* Errors and argument checks. A null array that a call reads or writes (when its length is not 0)
 * returns NPA_ERR_INVALID_ARGUMENT before any device work is queued. NPA_ERR_COORD_OVERFLOW:
 * a hashgrid build met a Particle-mode cell coordinate beyond +-2^30 (positions beyond about
 * 2^30 * eps), where the device path's i32 cell records are no longer exact. Device-pointer calls
 * queue their work without waiting, so the overflow of such a call is returned by the next call
 * on the same context (or, for a state, by npa_state_read) that synchronises: every call in
 * host-I/O mode, npa_neighbor_lists, npa_state_read, npa_state_pair_counts and
 * npa_context_synchronize. Reporting it clears it. */

/* ---------------------------------------------------------------- config */
/* Boundary / HashGridMode: crates/burn_automata_kernels/src/config.rs:4-18 */
enum { NPA_BOUNDARY_PERIODIC = 0, NPA_BOUNDARY_CLAMPED = 1 };
enum { NPA_MODE_GRID = 0, NPA_MODE_PARTICLE = 1 };

/* HashGridConfig: crates/burn_automata_kernels/src/config.rs:20-29 */
typedef struct npa_grid_cfg {
    uint32_t dim;          /* 2 or 3 */
    uint32_t boundary;     /* NPA_BOUNDARY_* */
    uint32_t mode;         /* NPA_MODE_* */
    uint32_t grid_size[3];
    float eps;             /* cell size == kernel support radius */
    uint32_t max_particles_per_block;  /* carried for fidelity; unused by the hot path */
} npa_grid_cfg;

/* PerceptionOptions: crates/burn_automata_kernels/src/reference/types.rs:4-15 (bools as u32) */
typedef struct npa_perception_opts {
    uint32_t state_grad;
    uint32_t density_grad;
    float eps0;
    uint32_t scale_equivariance;
    uint32_t particle_density_equivariance;
    uint32_t log_norm_grad;
    uint32_t log_norm_density_grad;
    uint32_t hybrid_state_gradient;
    uint32_t position_features;
} npa_perception_opts;

/* EquivarianceMode: crates/burn_automata/src/config.rs:22-28 */
enum { NPA_EQUIV_NONE = 0, NPA_EQUIV_PARTICLE_DENSITY = 1, NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE = 2 };

/* NpaConfig (the fields the rollout step reads): crates/burn_automata/src/config.rs:30-53 */
typedef struct npa_model_cfg {
    uint32_t spatial_dims;
    uint32_t state_dims;
    uint32_t hidden_dims;
    float eps0;
    float alpha;
    uint32_t density_grad;
    uint32_t state_grad;
    uint32_t log_norm_grad;
    uint32_t log_norm_density_grad;
    uint32_t equivariance;       /* NPA_EQUIV_* */
    uint32_t position_features;
} npa_model_cfg;

/* NpaWeights: crates/burn_automata/src/model.rs:12-17 (row-major) */
typedef struct npa_weights {
    const float* w1;   /* [H][F] */
    const float* b1;   /* [H]    */
    const float* w2;   /* [O][H] */
    const float* b2;   /* [O]    */
} npa_weights;

/* GaussianDecodeMode / GaussianDecodeConfig: crates/burn_automata_kernels/src/gaussian.rs:13-51 */
enum {
    NPA_DECODE_PARTICLE_POINT = 0,
    NPA_DECODE_SH0_FIXED_SCALE = 1,
    NPA_DECODE_SH0_LEARNED_SCALE = 2,
    NPA_DECODE_SH0_ORIENTED = 3
};
typedef struct npa_gaussian_decode_cfg {
    uint32_t mode;
    float sigma;
    float min_scale;
    float max_scale;
    float max_anisotropy;
    float opacity_scale;
    float min_opacity;
    float max_opacity;
    uint32_t sh_degree;
} npa_gaussian_decode_cfg;

/* Splat2dConfig: crates/burn_automata_kernels/src/splat.rs:6-14 */
typedef struct npa_splat2d_cfg {
    uint32_t image_size;
    float sigma;
    float lo;
    float hi;
    uint32_t normalize_color;
    uint32_t y_up;
    float pixel_size;
} npa_splat2d_cfg;

/* RenderViewPreset: crates/burn_automata/src/render_loss.rs:25-31 */
enum { NPA_VIEW_XY = 0, NPA_VIEW_XZ = 1, NPA_VIEW_YZ = 2, NPA_VIEW_ISO = 3 };

/* RenderLossConfig: crates/burn_automata/src/render_loss.rs:33-63 (reference defaults in
 * brackets). The raster reads image_size, the sigma fields, gaussian_decode_mode,
 * world_scale and opacity_logit_bias; the remaining fields are validated as the reference
 * validates them (render_loss/attributes.rs:114-174). */
typedef struct npa_render_cfg {
    uint32_t image_size;           /* [64] */
    float sigma;                   /* [2.5] pixels */
    float min_sigma;               /* [0.75] */
    float max_sigma;               /* [5.0] */
    uint32_t gaussian_decode_mode; /* NPA_DECODE_* [NPA_DECODE_SH0_FIXED_SCALE] */
    float world_scale;             /* [1.25] */
    uint32_t target_samples;       /* [8192] */
    float opacity_logit_bias;      /* [0.0] */
    float density_weight;          /* [1.0] */
    float color_weight;            /* [1.0] */
    float depth_weight;            /* [1.0] */
} npa_render_cfg;

/* ------------------------------------------------------------- context */
typedef struct npa_context npa_context;
typedef struct npa_state npa_state;

/* Creates a context bound to HIP device `device`. `stream` is a hipStream_t
 * (may be NULL for the legacy default stream); the context never destroys it. */
npa_status npa_context_create(int device, void* stream, npa_context** out);
/* Ends the caller's use of ctx. States created on it keep the context's memory alive: it is
 * released when the last of them is destroyed, in either order. The library never owns the
 * caller's stream: the caller keeps it valid until the last state of the context is destroyed
 * (state calls and that final release are queued on it). */
void npa_context_destroy(npa_context* ctx);
npa_status npa_context_set_stream(npa_context* ctx, void* stream);
/* 0: array arguments are device pointers (default). 1: host pointers, synchronous. */
npa_status npa_context_set_host_io(npa_context* ctx, int host_io);
/* Update-MLP engine of npa_step and of states (no counterpart in the reference, whose MLP is a
 * serial f32 loop). NPA_MLP_VALU (default): every sum in the reference's order on the vector
 * ALUs, bit-identical to the CPU path. NPA_MLP_MFMA: the two dense layers on the fp32 matrix
 * cores (v_mfma_f32_4x4x1f32 in the fused step kernel, v_mfma_f32_16x16x4_f32 otherwise), with
 * fused products and split sums: a single step stays within 1e-6 of the reference, while a
 * rollout drifts apart as far as the reference itself does from a one-ulp perturbation of its
 * inputs (the dynamics amplify last-bit differences). Measured on MI355X, the matrix-core engine's
 * step kernel is the faster one from 16,384 particles up; below that the VALU engine's is, as small
 * systems take four-wave blocks on that engine. NPA_MLP_MFMA_BF16: in the fused step kernel of 2D
 * systems, layer 1 on the bf16 matrix cores (v_mfma_f32_4x4x4bf16_1k) with each feature split into
 * three bf16 parts that sum to it exactly and the weights rounded to bf16: for bf16-valued weights
 * every product is exact and the step stays within the single-step gate; other weights are rounded
 * (relative error about 2^-9). Layer 2, 3D systems and the other kernels run as NPA_MLP_MFMA. */
enum { NPA_MLP_VALU = 0, NPA_MLP_MFMA = 1, NPA_MLP_MFMA_BF16 = 2 };
npa_status npa_context_set_mlp_engine(npa_context* ctx, int engine);

/* Blocks until all work queued on the context's stream has finished. */
npa_status npa_context_synchronize(npa_context* ctx);
/* Message of the last failing call on this context ("" when none). */
const char* npa_last_error(const npa_context* ctx);
/* Library version string. */
const char* npa_version(void);

/* ------------------------------------------------ operator surface (L0) */
/* Replaces build_hashgrid (crates/burn_automata_kernels/src/hashgrid.rs:16-69).
 * bin_offsets[B*C+1], permutation[B*N] (binned -> local particle index),
 * inverse_permutation[B*N] (global particle -> binned index - b*N).
 * Bit-exact with the reference's stable counting sort. */
npa_status npa_build_hashgrid(npa_context* ctx, const float* positions,
                              uint32_t batch_size, uint32_t particle_count,
                              const npa_grid_cfg* cfg,
                              uint32_t* bin_offsets, size_t bin_offsets_len,
                              uint32_t* permutation, uint32_t* inverse_permutation,
                              size_t particles_len);

/* Debug export of the ordered neighbour lists for_each_neighbor visits
 * (crates/burn_automata_kernels/src/reference/neighbor.rs:3-44), CSR form:
 * offsets[B*N+1], indices[capacity] (global particle indices, reference order).
 * When capacity is too small, only offsets are written and *required receives
 * the needed length. */
npa_status npa_neighbor_lists(npa_context* ctx, const float* positions,
                              uint32_t batch_size, uint32_t particle_count,
                              const npa_grid_cfg* cfg, uint32_t* offsets,
                              uint32_t* indices, size_t capacity, size_t* required);

/* Replaces perceive_with_options (crates/burn_automata_kernels/src/reference/forward.rs:26-143).
 * features[B*N][F]; density[B*N]; blurred_state[B*N][S];
 * state_gradient[B*N][S*d] (may be NULL; ignored when !state_grad);
 * density_gradient[B*N][d] (may be NULL; ignored when !density_grad).
 * *feature_dims receives F. */
npa_status npa_perceive(npa_context* ctx, const float* positions, const float* states,
                        uint32_t batch_size, uint32_t particle_count, uint32_t state_dims,
                        const npa_grid_cfg* cfg, const npa_perception_opts* opts,
                        float* features, size_t features_len, float* density,
                        float* blurred_state, float* state_gradient, float* density_gradient,
                        uint32_t* feature_dims);

/* Replaces perceive_adjoint_with_options
 * (crates/burn_automata_kernels/src/reference/adjoint.rs:27-136; perceive_state_adjoint_with_options
 * adjoint.rs:3-25 is its state half): the reverse mode of npa_perceive for the same positions,
 * states, grid and options. feature_adjoint[B*N][F] (feature_adjoint_len must equal B*N*F,
 * NPA_ERR_OUTPUT_SHAPE otherwise); state_adjoint[B*N][S]; position_adjoint[B*N][4] (w = 0; may be
 * NULL). Deterministic; equal to the reference up to the order of each particle's sums: the
 * reference scatters every pair's terms from idx into idx and j, this entry point gathers them
 * per particle over its own neighbour list (the relation is symmetric). */
npa_status npa_perceive_adjoint(npa_context* ctx, const float* positions, const float* states,
                                uint32_t batch_size, uint32_t particle_count, uint32_t state_dims,
                                const npa_grid_cfg* cfg, const npa_perception_opts* opts,
                                const float* feature_adjoint, size_t feature_adjoint_len,
                                float* state_adjoint, float* position_adjoint);

/* Replaces NpaModel::forward_from_features_with_eps
 * (crates/burn_automata/src/model.rs:867-940): update MLP, motion scaling.
 * features[rows][F] -> dx[rows][4] (axes >= d written as 0), ds[rows][S]. */
npa_status npa_mlp_forward(npa_context* ctx, const float* features, uint32_t rows,
                           const npa_model_cfg* model, const npa_weights* weights,
                           float eps, float* dx, float* ds);

/* Replaces euler_step (crates/burn_automata_kernels/src/reference/step.rs:4-55).
 * update_mask may be NULL (all ones). */
npa_status npa_euler_step(npa_context* ctx, const float* positions, const float* states,
                          const float* dx, const float* ds, uint32_t batch_size,
                          uint32_t particle_count, uint32_t state_dims,
                          const npa_grid_cfg* cfg, float dt, const float* update_mask,
                          float* out_positions, float* out_states);

/* Replaces NpaModel::step_cpu (crates/burn_automata/src/model.rs:768-858): one fused
 * rollout step. update_mask may be NULL (all ones); out_density may be NULL. */
npa_status npa_step(npa_context* ctx, const float* positions, const float* states,
                    uint32_t batch_size, uint32_t particle_count,
                    const npa_grid_cfg* grid, const npa_model_cfg* model,
                    const npa_weights* weights, float dt, const float* update_mask,
                    float* out_positions, float* out_states, float* out_density);

/* npa_step without any allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory - code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments, checks and results as npa_step (bit for bit), device pointers
 * only (NPA_ERR_INVALID_ARGUMENT in host-I/O mode); it calls no hipMalloc, hipFree, memset or
 * allocating library routine. Its workspace is a fixed device array of
 * NPA_STEP_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on until the process
 * ends; a system whose workspace does not fit is refused with NPA_ERR_INVALID_ARGUMENT before any
 * work is queued (the C2 system - 65,536 particles, S = 16, F = 64, a 64x64 grid - fits). Every
 * call on one GPU shares that array and the next call overwrites it: calls that overlap on one GPU
 * (on other streams, contexts or threads) race. The kernel profiler does not time it; its
 * coordinate overflows are reported by npa_context_synchronize of a context that has called it
 * (the overflow word is one per GPU, shared by every context there, not one per context). */
#define NPA_STEP_NOALLOC_SCRATCH_BYTES (64u << 20)
npa_status npa_step_noalloc(npa_context* ctx, const float* positions, const float* states,
                            uint32_t batch_size, uint32_t particle_count,
                            const npa_grid_cfg* grid, const npa_model_cfg* model,
                            const npa_weights* weights, float dt, const float* update_mask,
                            float* out_positions, float* out_states, float* out_density);

/* The device update mask of the reference GPU path (gpu_step.wgsl:1019-1056 with lane
 * seeds from crates/burn_automata/src/gpu/executor/state.rs:1282-1315):
 * mask[b*N+i] = random01(i, step_index, lane_seed(b)) < update_prob. */
npa_status npa_update_mask(npa_context* ctx, uint32_t batch_size, uint32_t particle_count,
                           float update_prob, uint32_t step_index, uint64_t seed,
                           float* mask);

/* Replaces decode_gaussians_3d (crates/burn_automata_kernels/src/gaussian.rs:53-100).
 * Planar outputs: position_visibility[n][4], spherical_harmonic[n][K][3] with
 * K = (sh_degree+1)^2 in oriented mode and 1 otherwise, rotation[n][4], scale_opacity[n][4]. */
npa_status npa_decode_gaussians_3d(npa_context* ctx, const float* positions,
                                   const float* states, uint32_t count, uint32_t state_dims,
                                   const npa_gaussian_decode_cfg* cfg,
                                   float* position_visibility, float* spherical_harmonic,
                                   float* rotation, float* scale_opacity);

/* Replaces splat_particles_2d (crates/burn_automata_kernels/src/splat.rs:30-93).
 * colors[count][3]; image[size*size][4] is overwritten. Tile-binned and
 * deterministic: each pixel sums particles in ascending index order. */
npa_status npa_splat_2d(npa_context* ctx, const float* positions, const float* colors,
                        uint32_t count, const npa_splat2d_cfg* cfg, float* image);

/* Batched systems drawn side by side (no counterpart in the reference, whose
 * splat_particles_2d draws one system; used for batched rollouts): system b of
 * batch_size systems of particle_count particles is drawn exactly as
 * splat_particles_2d draws it alone into an image_size-square window, placed at
 * window column b % tiles_x, row b / tiles_x. image[rows*size][tiles_x*size][4]
 * with rows = ceil(batch_size / tiles_x); windows past the last system are zero. */
npa_status npa_splat_2d_tiled(npa_context* ctx, const float* positions, const float* colors,
                              uint32_t batch_size, uint32_t particle_count,
                              const npa_splat2d_cfg* cfg, uint32_t tiles_x, float* image);

/* Replaces project_positions (crates/burn_automata/src/render_loss/projection.rs:11-29)
 * followed by splat_projected (render_loss/image.rs:18-79), once per view: image v is the
 * isotropic projected splat of all count particles seen through views[v] (NPA_VIEW_*, a
 * HOST array of nviews <= 16 entries). colors[count][3], opacities[count], sigmas[count]
 * (pixels; clamped to [min_sigma, max_sigma] by the splat). images[nviews][size][size][5]
 * holds RenderedPixel (image.rs:4-9): r, g, b, alpha, depth_sum; it is overwritten.
 * Deterministic; equal to the reference up to rounding: the weight is evaluated as
 * 2^(-d^2 log2(e) / 2 sigma^2) with one combined scale, the footprint weight sum is split over
 * 16 lanes, and a pixel adds its particles in ascending index order within chunks of 256,
 * the chunks in order. */
npa_status npa_render_views(npa_context* ctx, const float* positions, const float* colors,
                            const float* opacities, const float* sigmas, uint32_t count,
                            const uint32_t* views, uint32_t nviews, const npa_render_cfg* cfg,
                            float* images);

/* Replaces state_tail_render_attributes (render_loss/attributes.rs:15-87): per particle
 * colors[count][3] = clamp(tail + 0.5, 0, 1), opacities[count] (sigmoid of the material
 * opacity channel plus opacity_logit_bias, clamped to [0.001, 0.95]), sigmas[count] by the
 * decode mode, and scale_logit_derivatives[count] (may be NULL). */
npa_status npa_render_attributes(npa_context* ctx, const float* states, uint32_t count,
                                 uint32_t state_dims, const npa_render_cfg* cfg, float* colors,
                                 float* opacities, float* sigmas,
                                 float* scale_logit_derivatives);

/* ----------------------------------- device-resident executor (L2 twin) */
/* Replaces WgpuAutomataExecutor::create_state_with_update_prob
 * (crates/burn_automata/src/gpu/executor/state.rs:82-111). positions/states/weights
 * follow the context's I/O mode. The state owns ping-pong particle buffers and all
 * per-step workspaces; its first step has step index 0. */
npa_status npa_state_create(npa_context* ctx, const npa_model_cfg* model,
                            const npa_weights* weights, const npa_grid_cfg* grid,
                            const float* positions, const float* states,
                            uint32_t batch_size, uint32_t particle_count, float dt,
                            float update_prob, uint64_t seed, npa_state** out);
void npa_state_destroy(npa_state* state);
/* step_state / step_state_many (crates/burn_automata/src/gpu/executor/steps.rs:6-69). */
npa_status npa_state_step(npa_state* state, uint32_t steps);
/* read_state (crates/burn_automata/src/gpu/executor/readback.rs:85): current particles
 * and the density of the last step (density may be NULL). */
npa_status npa_state_read(npa_state* state, float* positions, float* states, float* density);
/* update_state_model (crates/burn_automata/src/gpu/executor/state.rs:626). */
npa_status npa_state_update_model(npa_state* state, const npa_weights* weights);
/* The state's update-MLP engine (NPA_MLP_*; see npa_context_set_mlp_engine). */
npa_status npa_state_set_mlp_engine(npa_state* state, int engine);
/* Current step index (number of steps taken). */
npa_status npa_state_step_index(const npa_state* state, uint64_t* step_index);
/* Device pointers of the current particle buffers (valid until the next step). */
npa_status npa_state_buffers(npa_state* state, float** positions, float** states);
/* Splat the current particles with colors clamp(state[S-3..S]+0.5, 0, 1)
 * (crates/burn_automata/examples/infer_2d.rs:20-39). image per context I/O mode. */
npa_status npa_state_splat_2d(npa_state* state, const npa_splat2d_cfg* cfg, float* image);
/* npa_splat_2d_tiled of the current particles, one window per system, colours as in
 * npa_state_splat_2d. */
npa_status npa_state_splat_2d_tiled(npa_state* state, const npa_splat2d_cfg* cfg, uint32_t tiles_x,
                                    float* image);
/* The particle images of mesh_multiview_render_loss_from_trace
 * (crates/burn_automata/src/render_loss.rs:107-141) for the current particles: the render
 * attributes of the current states (npa_render_attributes), then npa_render_views. The
 * reference renders batch-1 traces only (validate_render_trace, attributes.rs:89-112). */
npa_status npa_state_render_views(npa_state* state, const uint32_t* views, uint32_t nviews,
                                  const npa_render_cfg* cfg, float* images);
/* decode_gaussians_3d (gaussian.rs:53-100) of the current particles; the viewer's export is
 * npa_state_write_gaussians. */
npa_status npa_state_decode_gaussians_3d(npa_state* state, const npa_gaussian_decode_cfg* cfg,
                                         float* position_visibility, float* spherical_harmonic,
                                         float* rotation, float* scale_opacity);

/* ------------------------------------------------------- viewer export */
/* GAUSSIAN_SH_COEFF_COUNT (crates/burn_automata/src/gpu_step.wgsl:6): SH floats per Gaussian. */
#define NPA_GAUSSIAN_SH_COEFF_COUNT 48
/* Replaces write_state_into_gaussian_bind_group (crates/burn_automata/src/gpu/executor/steps.rs:71-108):
 * the planar Gaussian export the viewer reads (WgpuGaussianBufferRefs, crates/burn_automata/src/gpu/types.rs:55-60),
 * of the state's current particles, written by write_gaussian_from_output (gpu_step.wgsl:4963-5052):
 *   position_visibility[i] = (x, y, z (0 in 2D), 1);
 *   spherical_harmonic[i][48] = 0 except [0..3] = (clamp(tail + 0.5, 0, 1) - 0.5) / SH_C0, tail = the
 *     last three state channels (SH_C0 = 0.28209479177387814);
 *   rotation[i] = (1, 0, 0, 0) and scale_opacity[i].xyz = max(eps * 0.12, 8e-5); for 3D models with
 *     position features and S >= 9, the unit quaternion (w, x, y, z) taking +z onto the normal in
 *     channels 4..6 and a tangent-plane scale (t, t, max(0.18 t, 8e-5)),
 *     t = max(clamp(0.32 eps clamp(sqrt(4096 / N), 0.4, 2), 0.08 eps, 0.64 eps), 8e-5);
 *   scale_opacity[i].w = 1 in 2D, clamp(sigmoid(channel 8, or 3 when S <= 8), 0.001, 0.95) in 3D.
 * count is the capacity of the four arrays in Gaussians ([count][4], [count][48]): it must be at
 * least B*N (NPA_ERR_INVALID_ARGUMENT otherwise, as the reference); only the first B*N are written.
 * The reference's material branch (adaptive rollouts) is not part of this path. Deterministic; bit
 * for bit the oracle's restatement except the 3D opacity's exp (within 1e-6). */
npa_status npa_state_write_gaussians(npa_state* state, uint32_t count, float* position_visibility,
                                     float* spherical_harmonic, float* rotation, float* scale_opacity);
/* Replaces step_state_into_gaussians / step_state_many_into_gaussian_bind_group
 * (crates/burn_automata/src/gpu/executor/steps.rs:111-257): max(steps, 1) steps (as the reference,
 * 0 runs one), then the export of npa_state_write_gaussians of the particles the last step wrote. */
npa_status npa_state_step_into_gaussians(npa_state* state, uint32_t steps, uint32_t count,
                                         float* position_visibility, float* spherical_harmonic,
                                         float* rotation, float* scale_opacity);

/* ------------------------------------------------------- oriented Gaussian raster */
/* The EWA raster of the planar Gaussian export: the image the viewer draws from
 * decode_gaussians_3d / write_gaussian_main output through bevy_gaussian_splatting 8.0.1
 * (Cargo.toml:23; crates/bevy_automata/src/viewer/cloud.rs:80-97: 3D clouds, radix sort on
 * 32 depth bits). That crate is not vendored and no reference test pins its pixels, so this
 * restates the published 3D Gaussian splatting forward pass (Kerbl et al. 2023; the EWA
 * projection of Zwicker et al. 2001):
 *   camera frame: v = view * [p, 1] (camera looks down -z, +y up, as a bevy view matrix);
 *     depth z = -v.z; Gaussians with visibility <= 0, z <= near_plane or z > far_plane are culled;
 *   covariance: Sigma = R diag(s)^2 R^T from the unit quaternion (w, x, y, z) and scale s;
 *     Sigma2d = J W Sigma W^T J^T + 0.3 I (W: the view rotation with y and z flipped, J: the
 *     perspective Jacobian, its x/z and y/z clamped to 1.3x the image half-extent);
 *   footprint: the conic Sigma2d^-1 and radius ceil(3 sqrt(lambda_max)); the 16x16 pixel tiles
 *     within the radius of the centre (cx + fx x/z, cy + fy y'/z, y' = -v.y) list the Gaussian;
 *   colour: NPA_RASTER_COLOR_SH evaluates the real spherical harmonics of degree sh_degree at
 *     the direction from the camera centre (coefficients [n][(d+1)^2][3]) plus 0.5, floored at 0;
 *     NPA_RASTER_COLOR_RGB takes coefficient 0 as the colour (decode_gaussians_3d stores
 *     clamp(state + 0.5, 0, 1) there, gaussian.rs:133-157);
 *   compositing: each pixel (centre at +0.5) walks its tile's Gaussians front to back (depth
 *     ascending, ties by index): power = -(a dx^2 + c dy^2)/2 - b dx dy (skip when > 0),
 *     alpha = min(0.99, opacity e^power) (skip below 1/255); it stops before the Gaussian that
 *     would take transmittance T below 1e-4; rgb += colour alpha T, T *= 1 - alpha. The power is
 *     evaluated as qa dx^2 + qc dy^2 + qb dx dy with the conic pre-scaled by -log2(e)/2, -log2(e),
 *     -log2(e)/2 in fused multiply-adds, and e^power as 2^(that).
 * image[height][width][4] = premultiplied r, g, b and 1 - T; it is overwritten. */
enum { NPA_RASTER_COLOR_SH = 0, NPA_RASTER_COLOR_RGB = 1 };
typedef struct npa_raster_camera {
    float view[16];           /* row-major world -> camera */
    float fx, fy;             /* focal lengths, pixels */
    float cx, cy;             /* principal point, pixels from the top-left corner (y down) */
    uint32_t width, height;   /* pixels; at most 65536 16x16 tiles */
    float near_plane;         /* > 0 */
    float far_plane;          /* > near_plane */
    uint32_t sh_degree;       /* 0..3: (sh_degree+1)^2 coefficients per Gaussian */
    uint32_t color_mode;      /* NPA_RASTER_COLOR_* */
} npa_raster_camera;

npa_status npa_raster_gaussians_3d(npa_context* ctx, const float* position_visibility,
                                   const float* spherical_harmonic, const float* rotation,
                                   const float* scale_opacity, uint32_t count,
                                   const npa_raster_camera* camera, float* image);
/* The frame of a device-resident state, drawn by npa_raster_gaussians_3d from library-held buffers.
 * cfg NULL: the viewer's export (npa_state_write_gaussians) with its 48 SH coefficients, as
 * NPA_RASTER_COLOR_SH at degree 3 - the frame the viewer draws. cfg set: decode_gaussians_3d of the
 * current particles, whose coefficients are colours clamp(state + 0.5, 0, 1), read as
 * NPA_RASTER_COLOR_RGB from coefficient 0. camera->sh_degree and camera->color_mode are set by the
 * call in both cases. */
npa_status npa_state_raster_gaussians_3d(npa_state* state, const npa_gaussian_decode_cfg* cfg,
                                         const npa_raster_camera* camera, float* image);

/* ------------------------------------------------------- model files */
/* A BpkModelManifest (crates/burn_automata/src/import.rs:20-31) read from a .bpk container or
 * its bare JSON payload: replaces load_manifest / load_manifest_bytes (import.rs:378-390) and
 * decode_bpk_manifest (import.rs:460-498), with the same checks in the same order (header
 * length, magic, container version, payload length, SHA-256, JSON, validate_manifest
 * import.rs:500-506) and the same status per failure (NPA_ERR_INVALID_FORMAT, NPA_ERR_JSON,
 * NPA_ERR_INVALID_MODEL, NPA_ERR_IO). Host memory; no device is touched. The message of a
 * failure is written to err (err_len bytes, NUL-terminated) when err is not NULL. */
typedef struct npa_manifest npa_manifest;
npa_status npa_manifest_load(const uint8_t* bytes, size_t len, npa_manifest** out, char* err,
                             size_t err_len);
npa_status npa_manifest_load_file(const char* path, npa_manifest** out, char* err, size_t err_len);
void npa_manifest_destroy(npa_manifest* manifest);
/* Manifest header fields; strings stay valid until npa_manifest_destroy (source is NULL for
 * None; decoder_dims / output_dims are -1 for None). */
typedef struct npa_manifest_info_t {
    uint32_t format_version;
    const char* model_kind;
    const char* source;
    uint32_t auxiliary_input_dims;
    int64_t decoder_dims;
    int64_t output_dims;
    uint32_t stopgrad_pos;
    uint32_t stopgrad_state;
    uint32_t initialization_particles;  /* 0 when the manifest has no initialization */
} npa_manifest_info_t;
npa_status npa_manifest_info(const npa_manifest* manifest, npa_manifest_info_t* info);
/* BpkModelManifest::into_model (import.rs:94-99) as the ABI's config structs; weights point into
 * the manifest (host memory, valid until npa_manifest_destroy). NPA_ERR_INVALID_MODEL for a model
 * with auxiliary inputs, which the rollout path does not take. Any pointer may be NULL. */
npa_status npa_manifest_model(const npa_manifest* manifest, npa_model_cfg* model, npa_grid_cfg* grid,
                              npa_weights* weights);
/* The manifest's particle initialization (import.rs:33-37): positions[n][4], states[n][S];
 * NPA_ERR_INVALID_ARGUMENT when it has none. */
npa_status npa_manifest_initialization(const npa_manifest* manifest, const float** positions,
                                       const float** states, uint32_t* particle_count);
/* encode_bpk_manifest (import.rs:444-458) for an already serialized JSON payload: writes the
 * container (52-byte header + payload) to out; *required receives its length. out may be NULL to
 * query the length; NPA_ERR_OUTPUT_SHAPE when out_len is too small. */
npa_status npa_bpk_encode(const uint8_t* payload, size_t len, uint8_t* out, size_t out_len,
                          size_t* required);
/* SHA-256 (FIPS 180-4) of data, the container's checksum (sha2::Sha256 in the reference). */
npa_status npa_sha256(const uint8_t* data, size_t len, uint8_t* digest /* 32 bytes */);

/* ---------------------------------------------------------- profiling */
/* Kernel ids for npa_profile_read. */
enum {
    NPA_KERNEL_HASH_RANK = 0,
    NPA_KERNEL_TABLE_SCAN = 1,     /* hashgrid build: tile-column scan fused with the offsets scan */
    NPA_KERNEL_OFFSETS_SCAN = 2,   /* the separate offsets scan of the generic key sorts */
    NPA_KERNEL_SCATTER = 3,
    NPA_KERNEL_DENSITY = 4,
    NPA_KERNEL_PERCEIVE = 5,   /* second neighbour pass + normalisation + feature rows */
    NPA_KERNEL_SPLAT = 6,      /* the whole 2D splat pipeline */
    NPA_KERNEL_MLP = 7,        /* update MLP + masked Euler */
    NPA_KERNEL_SPLIT = 8,      /* per-bin split by true cell + sorted payload + work items + update-mask targets */
    NPA_KERNEL_ACTIVE = 9,     /* reserved: the split kernel (8) now selects the update-mask targets */
    NPA_KERNEL_RENDER = 10,    /* the whole projected 3D render pipeline (npa_render_views) */
    NPA_KERNEL_RASTER = 11,    /* the whole oriented Gaussian raster (npa_raster_gaussians_3d) */
    NPA_KERNEL_UPDATE = 12,    /* second neighbour pass + update MLP + masked Euler in one kernel (16-channel rows) */
    NPA_KERNEL_COUNT = 13
};
/* kernel_mask selects kernels by bit (1 << NPA_KERNEL_*; 0 = off, -1 = all). The
 * library then brackets each launch of a selected kernel with HIP events on the
 * context's stream. npa_profile_read synchronizes and returns the summed
 * milliseconds and launch count since the last reset. */
npa_status npa_profile_enable(npa_context* ctx, int kernel_mask);
npa_status npa_profile_reset(npa_context* ctx);
npa_status npa_profile_read(npa_context* ctx, int kernel_id, double* total_ms, uint64_t* launches);
/* Work counters of the state's next step on its current particles (exact, from the device;
 * diagnostic, no counterpart in the reference): candidates tested and pairs accepted by the
 * density pass over every particle, and the targets of the step's update mask (the particles the
 * second pass and the update MLP process) with their candidates and pairs. Any pointer may be
 * NULL. */
npa_status npa_state_pair_counts(npa_state* state, uint64_t* candidates, uint64_t* pairs, uint64_t* targets,
                                 uint64_t* target_candidates, uint64_t* target_pairs);

#ifdef __cplusplus
}
#endif

#endif /* NPA_ABI_H */
