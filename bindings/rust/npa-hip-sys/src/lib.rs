//! Raw `extern "C"` declarations of libnpa_hip.so (include/npa_abi.h), one for every entry point
//! and `#[repr(C)]` struct of the header, in the header's order and with its field order. Every
//! function returns an `npa_status` (`NPA_OK` = 0) unless the header says otherwise; pointers are
//! device pointers on a context in device-pointer mode and host pointers after
//! `npa_context_set_host_io(ctx, 1)`. The safe wrapper is the `npa-hip` crate.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void};

pub type npa_status = c_int;

pub const NPA_OK: npa_status = 0;
pub const NPA_ERR_INVALID_DIM: npa_status = 1;
pub const NPA_ERR_INVALID_EPS: npa_status = 2;
pub const NPA_ERR_INVALID_GRID_SIZE: npa_status = 3;
pub const NPA_ERR_PARTICLE_MODE_POW2: npa_status = 4;
pub const NPA_ERR_POSITION_SHAPE: npa_status = 10;
pub const NPA_ERR_STATE_SHAPE: npa_status = 11;
pub const NPA_ERR_OUTPUT_SHAPE: npa_status = 12;
pub const NPA_ERR_INVALID_ARGUMENT: npa_status = 13;
pub const NPA_ERR_INVALID_MODEL: npa_status = 20;
pub const NPA_ERR_IO: npa_status = 21;
pub const NPA_ERR_JSON: npa_status = 22;
pub const NPA_ERR_INVALID_FORMAT: npa_status = 23;
pub const NPA_ERR_DEVICE: npa_status = 30;
pub const NPA_ERR_OUT_OF_MEMORY: npa_status = 31;
pub const NPA_ERR_COORD_OVERFLOW: npa_status = 32;

pub const NPA_BOUNDARY_PERIODIC: u32 = 0;
pub const NPA_BOUNDARY_CLAMPED: u32 = 1;
pub const NPA_MODE_GRID: u32 = 0;
pub const NPA_MODE_PARTICLE: u32 = 1;
pub const NPA_EQUIV_NONE: u32 = 0;
pub const NPA_EQUIV_PARTICLE_DENSITY: u32 = 1;
pub const NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE: u32 = 2;
pub const NPA_DECODE_PARTICLE_POINT: u32 = 0;
pub const NPA_DECODE_SH0_FIXED_SCALE: u32 = 1;
pub const NPA_DECODE_SH0_LEARNED_SCALE: u32 = 2;
pub const NPA_DECODE_SH0_ORIENTED: u32 = 3;
pub const NPA_VIEW_XY: u32 = 0;
pub const NPA_VIEW_XZ: u32 = 1;
pub const NPA_VIEW_YZ: u32 = 2;
pub const NPA_VIEW_ISO: u32 = 3;
pub const NPA_MLP_VALU: c_int = 0;
pub const NPA_MLP_MFMA: c_int = 1;
pub const NPA_MLP_MFMA_BF16: c_int = 2;
pub const NPA_RASTER_COLOR_SH: u32 = 0;
pub const NPA_RASTER_COLOR_RGB: u32 = 1;
/// Kernel ids for npa_profile_enable (bit masks) and npa_profile_read.
pub const NPA_KERNEL_HASH_RANK: c_int = 0;
pub const NPA_KERNEL_TABLE_SCAN: c_int = 1;
pub const NPA_KERNEL_OFFSETS_SCAN: c_int = 2;
pub const NPA_KERNEL_SCATTER: c_int = 3;
pub const NPA_KERNEL_DENSITY: c_int = 4;
pub const NPA_KERNEL_PERCEIVE: c_int = 5;
pub const NPA_KERNEL_SPLAT: c_int = 6;
pub const NPA_KERNEL_MLP: c_int = 7;
pub const NPA_KERNEL_SPLIT: c_int = 8;
pub const NPA_KERNEL_ACTIVE: c_int = 9;
pub const NPA_KERNEL_RENDER: c_int = 10;
pub const NPA_KERNEL_RASTER: c_int = 11;
pub const NPA_KERNEL_UPDATE: c_int = 12;
pub const NPA_KERNEL_COUNT: c_int = 13;
pub const NPA_STEP_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;
pub const NPA_GAUSSIAN_SH_COEFF_COUNT: usize = 48;

/// HashGridConfig (crates/burn_automata_kernels/src/config.rs:20-29).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_grid_cfg {
    pub dim: u32,
    pub boundary: u32,
    pub mode: u32,
    pub grid_size: [u32; 3],
    pub eps: f32,
    pub max_particles_per_block: u32,
}

/// PerceptionOptions (crates/burn_automata_kernels/src/reference/types.rs:4-15), bools as u32.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_perception_opts {
    pub state_grad: u32,
    pub density_grad: u32,
    pub eps0: f32,
    pub scale_equivariance: u32,
    pub particle_density_equivariance: u32,
    pub log_norm_grad: u32,
    pub log_norm_density_grad: u32,
    pub hybrid_state_gradient: u32,
    pub position_features: u32,
}

/// NpaConfig, the fields the rollout step reads (crates/burn_automata/src/config.rs:30-53).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_model_cfg {
    pub spatial_dims: u32,
    pub state_dims: u32,
    pub hidden_dims: u32,
    pub eps0: f32,
    pub alpha: f32,
    pub density_grad: u32,
    pub state_grad: u32,
    pub log_norm_grad: u32,
    pub log_norm_density_grad: u32,
    pub equivariance: u32,
    pub position_features: u32,
}

/// NpaWeights (crates/burn_automata/src/model.rs:12-17), row-major w1 [H][F], w2 [O][H].
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct npa_weights {
    pub w1: *const f32,
    pub b1: *const f32,
    pub w2: *const f32,
    pub b2: *const f32,
}

/// GaussianDecodeConfig (crates/burn_automata_kernels/src/gaussian.rs:13-51).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_gaussian_decode_cfg {
    pub mode: u32,
    pub sigma: f32,
    pub min_scale: f32,
    pub max_scale: f32,
    pub max_anisotropy: f32,
    pub opacity_scale: f32,
    pub min_opacity: f32,
    pub max_opacity: f32,
    pub sh_degree: u32,
}

/// Splat2dConfig (crates/burn_automata_kernels/src/splat.rs:6-14).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_splat2d_cfg {
    pub image_size: u32,
    pub sigma: f32,
    pub lo: f32,
    pub hi: f32,
    pub normalize_color: u32,
    pub y_up: u32,
    pub pixel_size: f32,
}

/// RenderLossConfig (crates/burn_automata/src/render_loss.rs:33-63).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_render_cfg {
    pub image_size: u32,
    pub sigma: f32,
    pub min_sigma: f32,
    pub max_sigma: f32,
    pub gaussian_decode_mode: u32,
    pub world_scale: f32,
    pub target_samples: u32,
    pub opacity_logit_bias: f32,
    pub density_weight: f32,
    pub color_weight: f32,
    pub depth_weight: f32,
}

/// Camera of the oriented Gaussian raster (row-major world -> camera view matrix, pinhole).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct npa_raster_camera {
    pub view: [f32; 16],
    pub fx: f32,
    pub fy: f32,
    pub cx: f32,
    pub cy: f32,
    pub width: u32,
    pub height: u32,
    pub near_plane: f32,
    pub far_plane: f32,
    pub sh_degree: u32,
    pub color_mode: u32,
}

/// BpkModelManifest header fields (crates/burn_automata/src/import.rs:20-31).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct npa_manifest_info_t {
    pub format_version: u32,
    pub model_kind: *const c_char,
    pub source: *const c_char,
    pub auxiliary_input_dims: u32,
    pub decoder_dims: i64,
    pub output_dims: i64,
    pub stopgrad_pos: u32,
    pub stopgrad_state: u32,
    pub initialization_particles: u32,
}

#[repr(C)]
pub struct npa_context {
    _private: [u8; 0],
}
#[repr(C)]
pub struct npa_state {
    _private: [u8; 0],
}
#[repr(C)]
pub struct npa_manifest {
    _private: [u8; 0],
}

extern "C" {
    pub fn npa_context_create(device: c_int, stream: *mut c_void, out: *mut *mut npa_context) -> npa_status;
    pub fn npa_context_destroy(ctx: *mut npa_context);
    pub fn npa_context_set_stream(ctx: *mut npa_context, stream: *mut c_void) -> npa_status;
    pub fn npa_context_set_host_io(ctx: *mut npa_context, host_io: c_int) -> npa_status;
    pub fn npa_context_set_mlp_engine(ctx: *mut npa_context, engine: c_int) -> npa_status;
    pub fn npa_context_synchronize(ctx: *mut npa_context) -> npa_status;
    pub fn npa_last_error(ctx: *const npa_context) -> *const c_char;
    pub fn npa_version() -> *const c_char;

    pub fn npa_build_hashgrid(ctx: *mut npa_context, positions: *const f32, batch_size: u32, particle_count: u32,
                              cfg: *const npa_grid_cfg, bin_offsets: *mut u32, bin_offsets_len: usize,
                              permutation: *mut u32, inverse_permutation: *mut u32,
                              particles_len: usize) -> npa_status;
    pub fn npa_neighbor_lists(ctx: *mut npa_context, positions: *const f32, batch_size: u32, particle_count: u32,
                              cfg: *const npa_grid_cfg, offsets: *mut u32, indices: *mut u32, capacity: usize,
                              required: *mut usize) -> npa_status;
    pub fn npa_perceive(ctx: *mut npa_context, positions: *const f32, states: *const f32, batch_size: u32,
                        particle_count: u32, state_dims: u32, cfg: *const npa_grid_cfg,
                        opts: *const npa_perception_opts, features: *mut f32, features_len: usize,
                        density: *mut f32, blurred_state: *mut f32, state_gradient: *mut f32,
                        density_gradient: *mut f32, feature_dims: *mut u32) -> npa_status;
    pub fn npa_perceive_adjoint(ctx: *mut npa_context, positions: *const f32, states: *const f32, batch_size: u32,
                                particle_count: u32, state_dims: u32, cfg: *const npa_grid_cfg,
                                opts: *const npa_perception_opts, feature_adjoint: *const f32,
                                feature_adjoint_len: usize, state_adjoint: *mut f32,
                                position_adjoint: *mut f32) -> npa_status;
    pub fn npa_mlp_forward(ctx: *mut npa_context, features: *const f32, rows: u32, model: *const npa_model_cfg,
                           weights: *const npa_weights, eps: f32, dx: *mut f32, ds: *mut f32) -> npa_status;
    pub fn npa_euler_step(ctx: *mut npa_context, positions: *const f32, states: *const f32, dx: *const f32,
                          ds: *const f32, batch_size: u32, particle_count: u32, state_dims: u32,
                          cfg: *const npa_grid_cfg, dt: f32, update_mask: *const f32, out_positions: *mut f32,
                          out_states: *mut f32) -> npa_status;
    pub fn npa_step(ctx: *mut npa_context, positions: *const f32, states: *const f32, batch_size: u32,
                    particle_count: u32, grid: *const npa_grid_cfg, model: *const npa_model_cfg,
                    weights: *const npa_weights, dt: f32, update_mask: *const f32, out_positions: *mut f32,
                    out_states: *mut f32, out_density: *mut f32) -> npa_status;
    pub fn npa_step_noalloc(ctx: *mut npa_context, positions: *const f32, states: *const f32, batch_size: u32,
                            particle_count: u32, grid: *const npa_grid_cfg, model: *const npa_model_cfg,
                            weights: *const npa_weights, dt: f32, update_mask: *const f32,
                            out_positions: *mut f32, out_states: *mut f32, out_density: *mut f32) -> npa_status;
    pub fn npa_update_mask(ctx: *mut npa_context, batch_size: u32, particle_count: u32, update_prob: f32,
                           step_index: u32, seed: u64, mask: *mut f32) -> npa_status;
    pub fn npa_decode_gaussians_3d(ctx: *mut npa_context, positions: *const f32, states: *const f32, count: u32,
                                   state_dims: u32, cfg: *const npa_gaussian_decode_cfg,
                                   position_visibility: *mut f32, spherical_harmonic: *mut f32,
                                   rotation: *mut f32, scale_opacity: *mut f32) -> npa_status;
    pub fn npa_splat_2d(ctx: *mut npa_context, positions: *const f32, colors: *const f32, count: u32,
                        cfg: *const npa_splat2d_cfg, image: *mut f32) -> npa_status;
    pub fn npa_splat_2d_tiled(ctx: *mut npa_context, positions: *const f32, colors: *const f32, batch_size: u32,
                              particle_count: u32, cfg: *const npa_splat2d_cfg, tiles_x: u32,
                              image: *mut f32) -> npa_status;
    pub fn npa_render_views(ctx: *mut npa_context, positions: *const f32, colors: *const f32,
                            opacities: *const f32, sigmas: *const f32, count: u32, views: *const u32, nviews: u32,
                            cfg: *const npa_render_cfg, images: *mut f32) -> npa_status;
    pub fn npa_render_attributes(ctx: *mut npa_context, states: *const f32, count: u32, state_dims: u32,
                                 cfg: *const npa_render_cfg, colors: *mut f32, opacities: *mut f32,
                                 sigmas: *mut f32, scale_logit_derivatives: *mut f32) -> npa_status;

    pub fn npa_state_create(ctx: *mut npa_context, model: *const npa_model_cfg, weights: *const npa_weights,
                            grid: *const npa_grid_cfg, positions: *const f32, states: *const f32, batch_size: u32,
                            particle_count: u32, dt: f32, update_prob: f32, seed: u64,
                            out: *mut *mut npa_state) -> npa_status;
    pub fn npa_state_destroy(state: *mut npa_state);
    pub fn npa_state_step(state: *mut npa_state, steps: u32) -> npa_status;
    pub fn npa_state_read(state: *mut npa_state, positions: *mut f32, states: *mut f32, density: *mut f32) -> npa_status;
    pub fn npa_state_update_model(state: *mut npa_state, weights: *const npa_weights) -> npa_status;
    pub fn npa_state_set_mlp_engine(state: *mut npa_state, engine: c_int) -> npa_status;
    pub fn npa_state_step_index(state: *const npa_state, step_index: *mut u64) -> npa_status;
    pub fn npa_state_buffers(state: *mut npa_state, positions: *mut *mut f32, states: *mut *mut f32) -> npa_status;
    pub fn npa_state_splat_2d(state: *mut npa_state, cfg: *const npa_splat2d_cfg, image: *mut f32) -> npa_status;
    pub fn npa_state_splat_2d_tiled(state: *mut npa_state, cfg: *const npa_splat2d_cfg, tiles_x: u32,
                                    image: *mut f32) -> npa_status;
    pub fn npa_state_render_views(state: *mut npa_state, views: *const u32, nviews: u32, cfg: *const npa_render_cfg,
                                  images: *mut f32) -> npa_status;
    pub fn npa_state_decode_gaussians_3d(state: *mut npa_state, cfg: *const npa_gaussian_decode_cfg,
                                         position_visibility: *mut f32, spherical_harmonic: *mut f32,
                                         rotation: *mut f32, scale_opacity: *mut f32) -> npa_status;
    pub fn npa_state_write_gaussians(state: *mut npa_state, count: u32, position_visibility: *mut f32,
                                     spherical_harmonic: *mut f32, rotation: *mut f32,
                                     scale_opacity: *mut f32) -> npa_status;
    pub fn npa_state_step_into_gaussians(state: *mut npa_state, steps: u32, count: u32,
                                         position_visibility: *mut f32, spherical_harmonic: *mut f32,
                                         rotation: *mut f32, scale_opacity: *mut f32) -> npa_status;
    pub fn npa_raster_gaussians_3d(ctx: *mut npa_context, position_visibility: *const f32,
                                   spherical_harmonic: *const f32, rotation: *const f32,
                                   scale_opacity: *const f32, count: u32, camera: *const npa_raster_camera,
                                   image: *mut f32) -> npa_status;
    pub fn npa_state_raster_gaussians_3d(state: *mut npa_state, cfg: *const npa_gaussian_decode_cfg,
                                         camera: *const npa_raster_camera, image: *mut f32) -> npa_status;

    pub fn npa_manifest_load(bytes: *const u8, len: usize, out: *mut *mut npa_manifest, err: *mut c_char,
                             err_len: usize) -> npa_status;
    pub fn npa_manifest_load_file(path: *const c_char, out: *mut *mut npa_manifest, err: *mut c_char,
                                  err_len: usize) -> npa_status;
    pub fn npa_manifest_destroy(manifest: *mut npa_manifest);
    pub fn npa_manifest_info(manifest: *const npa_manifest, info: *mut npa_manifest_info_t) -> npa_status;
    pub fn npa_manifest_model(manifest: *const npa_manifest, model: *mut npa_model_cfg, grid: *mut npa_grid_cfg,
                              weights: *mut npa_weights) -> npa_status;
    pub fn npa_manifest_initialization(manifest: *const npa_manifest, positions: *mut *const f32,
                                       states: *mut *const f32, particle_count: *mut u32) -> npa_status;
    pub fn npa_bpk_encode(payload: *const u8, len: usize, out: *mut u8, out_len: usize,
                          required: *mut usize) -> npa_status;
    pub fn npa_sha256(data: *const u8, len: usize, digest: *mut u8) -> npa_status;

    pub fn npa_profile_enable(ctx: *mut npa_context, kernel_mask: c_int) -> npa_status;
    pub fn npa_profile_reset(ctx: *mut npa_context) -> npa_status;
    pub fn npa_profile_read(ctx: *mut npa_context, kernel_id: c_int, total_ms: *mut f64, launches: *mut u64) -> npa_status;
    pub fn npa_state_pair_counts(state: *mut npa_state, candidates: *mut u64, pairs: *mut u64, targets: *mut u64,
                                 target_candidates: *mut u64, target_pairs: *mut u64) -> npa_status;
}
