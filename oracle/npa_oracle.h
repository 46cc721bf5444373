/*
 * npa_oracle.h - CPU restatement of burn_automata's fixed-NPA rollout path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path and
 * the "port" CPU baseline; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product library (libnpa_hip.so) never calls it.
 *
 * Each function follows the reference Rust source cited beside it, operation
 * by operation (same association order, no FMA contraction: build with
 * -ffp-contract=off). Per-particle loops run under OpenMP like the reference's
 * rayon loops; every per-particle sum stays serial in neighbour order, so the
 * results do not depend on the thread count.
 *
 * Parity pinning (what checks each function beyond the restatement itself):
 *   hashgrid / cell hash      - reference test hashgrid_counts_particles_per_cell,
 *                               brute-force stable sort, permutation invariants
 *   neighbour lists           - all-pairs brute force (same set), order rule
 *   perceive (both branches)  - known-answer test perceive_matches_upstream_sph_kernel_constants,
 *                               poly6 normalisation integral, linear-field gradient,
 *                               scale equivariance (equivariance.rs), branch A/B agreement
 *   MLP / forward             - integer-weight closed forms
 *   euler_step                - reference tests euler_step_applies_masks_and_boundaries,
 *                               euler_step_clamps_3d_opacity_logit
 *   update mask               - p=0/p=1 limits, Bernoulli mean, lane-seed structure
 *   decode_gaussians_3d       - reference tests splat_and_gaussian_decode_are_shape_stable,
 *                               gaussian_decode_modes_cover_fixed_learned_and_oriented_scale
 *   splat_particles_2d        - closed-form single-particle Gaussian, additivity
 *   write_gaussians           - the reference's export tests (tests/gpu_wgpu/gaussian.rs:243-310:
 *                               position, visibility, identity rotation, positive scale, opacity
 *                               range), SH DC decoding back to the clamped colour
 *                               (SH_C0 * dc + 0.5), the normal branch's quaternion rotating +z onto
 *                               the unit normal (and the antipodal case), tangent scale and
 *                               opacity against float64 closed forms and scipy's expit
 *   view_basis / project_positions / splat_projected / render attributes
 *                             - orthonormal right-handed bases, axis views by coordinate
 *                               permutation, single-particle moments (total alpha = opacity,
 *                               centroid = projected pixel, second moment = sigma^2,
 *                               depth_sum / alpha = depth), sigmoid against scipy's expit,
 *                               reference test constants (RENDER_MIN/MAX_OPACITY, defaults)
 *   raster_gaussians_3d       - parity unpinned against the reference (its raster lives in the
 *                               un-vendored bevy_gaussian_splatting); pinned by closed forms: a
 *                               centred isotropic Gaussian's alpha profile, rotation invariance of
 *                               isotropic Gaussians, axis swaps of anisotropic ones, the analytic
 *                               conic of a rotated ellipse, two-layer compositing order, the
 *                               transmittance cut, SH bases against scipy's spherical harmonics
 *   perceive_adjoint          - the reference's finite-difference tests (lib.rs:123-356) with their
 *                               fixtures and tolerances; central differences of the oracle's
 *                               forward at every state and position coordinate of small systems;
 *                               linearity in the feature adjoint; identity and position-feature
 *                               rows
 */
#ifndef NPA_ORACLE_H
#define NPA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/npa_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

int oracle_grid_validate(const npa_grid_cfg* cfg);
uint32_t oracle_cell_count(const npa_grid_cfg* cfg);
void oracle_cell_coords(const float* pos4, const npa_grid_cfg* cfg, int64_t coords[3]);
uint32_t oracle_cell_for_position(const float* pos4, const npa_grid_cfg* cfg);

int oracle_build_hashgrid(const float* positions, uint32_t batch_size, uint32_t particle_count,
                          const npa_grid_cfg* cfg, uint32_t* bin_offsets, uint32_t* permutation,
                          uint32_t* inverse_permutation);

/* CSR neighbour lists in for_each_neighbor order; returns the total length or
 * (size_t)-1 on a config error. indices may be NULL to query the length. */
size_t oracle_neighbor_lists(const float* positions, uint32_t batch_size, uint32_t particle_count,
                             const npa_grid_cfg* cfg, uint32_t* offsets, uint32_t* indices);

uint32_t oracle_feature_dims(uint32_t state_dims, uint32_t dim, const npa_perception_opts* opts);

/* perceive_with_options. state_gradient / density_gradient may be NULL. */
int oracle_perceive(const float* positions, const float* states, uint32_t batch_size,
                    uint32_t particle_count, uint32_t state_dims, const npa_grid_cfg* cfg,
                    const npa_perception_opts* opts, float* features, float* density,
                    float* blurred_state, float* state_gradient, float* density_gradient);

void oracle_perception_opts_for_model(const npa_model_cfg* model, npa_perception_opts* out);
uint32_t oracle_model_perception_dims(const npa_model_cfg* model);

/* forward_update_from_features: update[rows][O] */
int oracle_forward_update(const float* features, uint32_t rows, const npa_model_cfg* model,
                          const npa_weights* weights, float* update);
/* forward_from_features_with_eps: dx[rows][4], ds[rows][S] */
int oracle_forward_from_features(const float* features, uint32_t rows,
                                 const npa_model_cfg* model, const npa_weights* weights,
                                 float eps, float* dx, float* ds);

int oracle_euler_step(const float* positions, const float* states, const float* dx,
                      const float* ds, uint32_t batch_size, uint32_t particle_count,
                      uint32_t state_dims, const npa_grid_cfg* cfg, float dt,
                      const float* update_mask, float* out_positions, float* out_states);

/* NpaModel::step_cpu. features/density/dx/ds outputs may be NULL. */
int oracle_step(const float* positions, const float* states, uint32_t batch_size,
                uint32_t particle_count, const npa_grid_cfg* grid, const npa_model_cfg* model,
                const npa_weights* weights, float dt, const float* update_mask,
                float* out_positions, float* out_states, float* out_density, float* out_dx,
                float* out_ds);

/* Sampled evaluation for systems too large for a full pass: the density of particles
 * sel[0..rows) only, and one step_cpu of those particles given every particle's density
 * (rows 0..rows of the outputs). */
int oracle_density_rows(const float* positions, uint32_t batch_size, uint32_t particle_count,
                        const npa_grid_cfg* cfg, const uint32_t* sel, uint64_t rows,
                        float* density);
int oracle_step_rows(const float* positions, const float* states, uint32_t batch_size,
                     uint32_t particle_count, const npa_grid_cfg* grid, const npa_model_cfg* model,
                     const npa_weights* weights, float dt, const float* update_mask,
                     const float* density, const uint32_t* sel, uint64_t rows,
                     float* out_positions, float* out_states);

uint32_t oracle_hash_u32(uint32_t value);
float oracle_random01(uint32_t particle, uint32_t step, uint32_t seed);
uint32_t oracle_gpu_random_seed(uint64_t seed);
void oracle_update_mask(uint32_t batch_size, uint32_t particle_count, float update_prob,
                        uint32_t step_index, uint64_t seed, float* mask);

/* Rollout with the device hash mask, step indices start_step .. start_step+steps-1.
 * positions/states are updated in place. */
int oracle_rollout(float* positions, float* states, uint32_t batch_size, uint32_t particle_count,
                   const npa_grid_cfg* grid, const npa_model_cfg* model,
                   const npa_weights* weights, float dt, float update_prob, uint64_t seed,
                   uint32_t start_step, uint32_t steps);

uint32_t oracle_decode_sh_coeffs(const npa_gaussian_decode_cfg* cfg);
int oracle_decode_gaussians_3d(const float* positions, const float* states, uint32_t count,
                               uint32_t state_dims, const npa_gaussian_decode_cfg* cfg,
                               float* position_visibility, float* spherical_harmonic,
                               float* rotation, float* scale_opacity);

/* write_gaussian_from_output (gpu_step.wgsl:4963-5052): pos_vis [total][4], sh [total][48],
 * rotation [total][4], scale_opacity [total][4]. */
int oracle_write_gaussians(const float* positions, const float* states, uint64_t total, uint32_t particle_count,
                           uint32_t S, uint32_t dim, float eps, int position_features, float* pos_vis, float* sh,
                           float* rotation, float* scale_opacity);
int oracle_splat_particles_2d(const float* positions, const float* colors, uint32_t count,
                              const npa_splat2d_cfg* cfg, float* image);

/* 3D render raster (crates/burn_automata/src/render_loss/): view_basis, project_positions
 * (projected[count][3] = x, y, depth), splat_projected (image[size*size][5] = r, g, b, alpha,
 * depth_sum) and state_tail_render_attributes (derivatives may be NULL). */
int oracle_view_basis(uint32_t view, float right[3], float up[3], float forward[3]);
int oracle_project_positions(uint32_t view, const float* positions, uint32_t count, float world_scale,
                             float* projected);
int oracle_splat_projected(const float* projected, const float* colors, const float* opacities,
                           const float* sigmas, uint32_t count, const npa_render_cfg* cfg, float* image);
int oracle_render_attributes(const float* states, uint32_t count, uint32_t state_dims, const npa_render_cfg* cfg,
                             float* colors, float* opacities, float* sigmas, float* derivatives);

/* perceive_adjoint_with_options (crates/burn_automata_kernels/src/reference/adjoint.rs:27-136):
 * feature_adjoint [total][F] -> state_adjoint [total][S], position_adjoint [total][4]. */
int oracle_perceive_adjoint(const float* positions, const float* states, uint32_t batch_size,
                            uint32_t particle_count, uint32_t state_dims, const npa_grid_cfg* cfg,
                            const npa_perception_opts* opts, const float* feature_adjoint,
                            float* state_adjoint, float* position_adjoint);

/* EWA raster of oriented 3D Gaussians (npa_raster_gaussians_3d's definition; the reference's
 * bevy_gaussian_splatting raster is not vendored): image[height][width][4]; *evaluated (may be
 * NULL) receives the number of (pixel, Gaussian) evaluations before each pixel's stop. */
int oracle_raster_camera_center(const npa_raster_camera* cam, float out[3]);
int oracle_raster_gaussians_3d(const float* position_visibility, const float* spherical_harmonic,
                               const float* rotation, const float* scale_opacity, uint32_t count,
                               const npa_raster_camera* cam, float* image, uint64_t* evaluated);

/* Per-phase wall-clock seconds of the last oracle_step / oracle_rollout call
 * (hashgrid+perceive, MLP+gates+integrate, 0), following profile_rollout
 * (crates/burn_automata/src/cli/bench.rs:652-722). */
void oracle_last_phase_seconds(double* perceive, double* mlp, double* integrate);
int oracle_max_threads(void);
void oracle_set_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif
