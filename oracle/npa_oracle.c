/*
 * npa_oracle.c - CPU restatement of burn_automata's fixed-NPA rollout path.
 *
 * TEST INFRASTRUCTURE ONLY (checker + "port" CPU baseline); see npa_oracle.h.
 * Build: gcc -O3 -fopenmp -ffp-contract=off (no fast-math), see oracle/Makefile.
 *
 * Every function cites the reference file:line it restates. Float expressions
 * keep the reference's left-to-right association; Rust never contracts a*b+c
 * into an FMA, so neither does this file.
 */
#include "npa_oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define PI_F 3.14159265358979323846f /* std::f32::consts::PI */

static double g_phase_perceive, g_phase_mlp, g_phase_integrate;

void oracle_last_phase_seconds(double* perceive, double* mlp, double* integrate) {
    if (perceive) *perceive = g_phase_perceive;
    if (mlp) *mlp = g_phase_mlp;
    if (integrate) *integrate = g_phase_integrate;
}

int oracle_max_threads(void) { return omp_get_max_threads(); }
void oracle_set_threads(int threads) {
    if (threads > 0) omp_set_num_threads(threads);
}

/* f32::powi with a non-negative exponent: LLVM expands llvm.powi with a constant
 * exponent into the square-and-multiply tree below, and compiler-rt's __powisf2
 * runs the same recurrence for a runtime exponent, so both give this value. */
static float powi_f32(float x, int n) {
    int recip = n < 0;
    unsigned b = (unsigned)(recip ? -n : n);
    float r = 1.0f;
    for (;;) {
        if (b & 1u) r *= x;
        b >>= 1;
        if (b == 0) break;
        x *= x;
    }
    return recip ? 1.0f / r : r;
}

/* `f as isize` for a floored f32: saturating, NaN -> 0 (Rust float->int cast). */
static int64_t f32_to_isize(float f) {
    if (isnan(f)) return 0;
    if (f >= 9223372036854775808.0f) return INT64_MAX;
    if (f <= -9223372036854775808.0f) return INT64_MIN;
    return (int64_t)f;
}

static int64_t rem_euclid_i64(int64_t a, int64_t m) {
    int64_t r = a % m;
    return r < 0 ? r + m : r;
}

static float rem_euclid_f32(float a, float m) {
    float r = fmodf(a, m);
    return r < 0.0f ? r + fabsf(m) : r;
}

static float clamp_f32(float v, float lo, float hi) { /* f32::clamp */
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* ---------------------------------------------------------------- config */

/* HashGridConfig::validate  crates/burn_automata_kernels/src/config.rs:65-84 */
int oracle_grid_validate(const npa_grid_cfg* cfg) {
    if (!(cfg->dim == 2 || cfg->dim == 3)) return NPA_ERR_INVALID_DIM;
    if (!isfinite(cfg->eps) || cfg->eps <= 0.0f) return NPA_ERR_INVALID_EPS;
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        uint32_t s = cfg->grid_size[a];
        if (s == 0) return NPA_ERR_INVALID_GRID_SIZE;
        if (cfg->mode == NPA_MODE_PARTICLE && (s & (s - 1u)) != 0) return NPA_ERR_PARTICLE_MODE_POW2;
    }
    return NPA_OK;
}

/* HashGridConfig::cell_count  config.rs:86-88 */
uint32_t oracle_cell_count(const npa_grid_cfg* cfg) {
    uint32_t c = 1;
    for (uint32_t a = 0; a < cfg->dim; ++a) c *= cfg->grid_size[a];
    return c;
}

static int spatial_mem_dims(const npa_grid_cfg* cfg) { return cfg->dim == 3 ? 4 : 2; } /* config.rs:90-92 */

/* ---------------------------------------------------------------- hashgrid */

/* mix_coord  crates/burn_automata_kernels/src/hashgrid.rs:155-163 */
static uint32_t mix_coord(int64_t value, uint32_t salt) {
    uint32_t x = ((uint32_t)(int32_t)value) ^ salt;
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

/* particle_cell_hash  hashgrid.rs:147-153 */
static uint32_t particle_cell_hash(const int64_t coords[3], const npa_grid_cfg* cfg) {
    uint32_t h = mix_coord(coords[0], 0x9e3779b9u) ^ mix_coord(coords[1], 0x85ebca6bu);
    if (cfg->dim == 3) h ^= mix_coord(coords[2], 0xc2b2ae35u);
    return (uint32_t)((uint64_t)h % (uint64_t)oracle_cell_count(cfg));
}

/* cell_coords_for_position  hashgrid.rs:98-121 */
void oracle_cell_coords(const float* p, const npa_grid_cfg* cfg, int64_t coords[3]) {
    coords[0] = coords[1] = coords[2] = 0;
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        if (cfg->mode == NPA_MODE_PARTICLE) {
            coords[a] = f32_to_isize(floorf(p[a] / cfg->eps));
            continue;
        }
        int64_t size = (int64_t)cfg->grid_size[a];
        float extent = cfg->eps * (float)cfg->grid_size[a];
        float half = extent * 0.5f;
        int64_t cell = f32_to_isize(floorf((p[a] + half) / cfg->eps));
        if (cfg->boundary == NPA_BOUNDARY_PERIODIC) {
            cell = rem_euclid_i64(cell, size);
        } else {
            if (cell < 0) cell = 0;
            if (cell > size - 1) cell = size - 1;
        }
        coords[a] = cell;
    }
}

/* cell_index_from_coords  hashgrid.rs:123-145; returns 0 for None */
static int cell_index_from_coords(const int64_t coords[3], const npa_grid_cfg* cfg, uint32_t* out) {
    if (cfg->mode == NPA_MODE_PARTICLE) {
        *out = particle_cell_hash(coords, cfg);
        return 1;
    }
    uint64_t stride = 1, hash = 0;
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        int64_t size = (int64_t)cfg->grid_size[a];
        int64_t cell;
        if (cfg->boundary == NPA_BOUNDARY_PERIODIC) {
            cell = rem_euclid_i64(coords[a], size);
        } else {
            if (coords[a] < 0 || coords[a] >= size) return 0;
            cell = coords[a];
        }
        hash += (uint64_t)cell * stride;
        stride *= (uint64_t)size;
    }
    *out = (uint32_t)hash;
    return 1;
}

/* cell_for_position  hashgrid.rs:71-96 */
uint32_t oracle_cell_for_position(const float* p, const npa_grid_cfg* cfg) {
    int64_t coords[3];
    if (cfg->mode == NPA_MODE_PARTICLE) {
        oracle_cell_coords(p, cfg, coords);
        return particle_cell_hash(coords, cfg);
    }
    uint64_t stride = 1, hash = 0;
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        int64_t size = (int64_t)cfg->grid_size[a];
        float extent = cfg->eps * (float)cfg->grid_size[a];
        float half = extent * 0.5f;
        int64_t cell = f32_to_isize(floorf((p[a] + half) / cfg->eps));
        if (cfg->boundary == NPA_BOUNDARY_PERIODIC) {
            cell = rem_euclid_i64(cell, size);
        } else {
            if (cell < 0) cell = 0;
            if (cell > size - 1) cell = size - 1;
        }
        hash += (uint64_t)cell * stride;
        stride *= (uint64_t)size;
    }
    return (uint32_t)hash;
}

/* build_hashgrid  hashgrid.rs:16-69 (serial stable counting sort, as in the reference) */
int oracle_build_hashgrid(const float* positions, uint32_t batch_size, uint32_t particle_count,
                          const npa_grid_cfg* cfg, uint32_t* bin_offsets, uint32_t* permutation,
                          uint32_t* inverse_permutation) {
    int st = oracle_grid_validate(cfg);
    if (st) return st;
    const uint64_t cells = oracle_cell_count(cfg);
    const uint64_t bins = (uint64_t)batch_size * cells;
    uint32_t* counts = (uint32_t*)calloc(bins ? bins : 1, sizeof(uint32_t));
    if (!counts) return NPA_ERR_OUT_OF_MEMORY;
    for (uint64_t b = 0; b < batch_size; ++b)
        for (uint64_t i = 0; i < particle_count; ++i) {
            uint64_t idx = b * particle_count + i;
            counts[b * cells + oracle_cell_for_position(positions + 4 * idx, cfg)] += 1;
        }
    bin_offsets[0] = 0;
    for (uint64_t k = 0; k < bins; ++k) bin_offsets[k + 1] = bin_offsets[k] + counts[k];
    /* write_heads = bin_offsets.clone() */
    for (uint64_t k = 0; k < bins; ++k) counts[k] = bin_offsets[k];
    for (uint64_t b = 0; b < batch_size; ++b)
        for (uint64_t i = 0; i < particle_count; ++i) {
            uint64_t idx = b * particle_count + i;
            uint64_t bin = b * cells + oracle_cell_for_position(positions + 4 * idx, cfg);
            uint32_t dst = counts[bin]++;
            permutation[dst] = (uint32_t)i;
            inverse_permutation[idx] = (uint32_t)(dst - b * particle_count);
        }
    free(counts);
    return NPA_OK;
}

/* ------------------------------------------------------------ neighbours */

typedef struct neighbor {
    uint32_t j;
    float delta[4];
    float r2;
} neighbor;

typedef struct nbuf {
    neighbor* v;
    size_t len, cap;
} nbuf;

static void nbuf_push(nbuf* b, uint32_t j, const float d[4], float r2) {
    if (b->len == b->cap) {
        b->cap = b->cap ? 2 * b->cap : 256;
        b->v = (neighbor*)realloc(b->v, b->cap * sizeof(neighbor));
    }
    neighbor* n = &b->v[b->len++];
    n->j = j;
    memcpy(n->delta, d, sizeof(n->delta));
    n->r2 = r2;
}

/* neighbor_delta  hashgrid.rs:165-181 */
static void neighbor_delta(const float* lhs, const float* rhs, const npa_grid_cfg* cfg, float d[4]) {
    d[0] = d[1] = d[2] = d[3] = 0.0f;
    for (uint32_t a = 0; a < cfg->dim; ++a) {
        float v = rhs[a] - lhs[a];
        if (cfg->boundary == NPA_BOUNDARY_PERIODIC) {
            float extent = (float)cfg->grid_size[a] * cfg->eps;
            float half = extent * 0.5f;
            if (v > half) v -= extent;
            else if (v < -half) v += extent;
        }
        d[a] = v;
    }
}

typedef struct grid_view {
    const uint32_t* bin_offsets;
    const uint32_t* permutation;
    uint32_t particle_count;
    uint32_t cell_count;
} grid_view;

/* for_each_neighbor  crates/burn_automata_kernels/src/reference/neighbor.rs:3-44
 * (collects the visited (j, delta, r2) triples in visit order) */
static void collect_neighbors(uint64_t idx, const float* positions, const grid_view* g,
                              const npa_grid_cfg* cfg, nbuf* out) {
    out->len = 0;
    const uint64_t batch = idx / g->particle_count;
    const uint64_t base = batch * g->particle_count;
    const float* pi = positions + 4 * idx;
    int64_t center[3];
    oracle_cell_coords(pi, cfg, center);
    const int zmin = cfg->dim == 3 ? -1 : 0, zmax = cfg->dim == 3 ? 1 : 0;
    const float eps2 = cfg->eps * cfg->eps;
    for (int dz = zmin; dz <= zmax; ++dz)
        for (int dy = -1; dy <= 1; ++dy)
            for (int dx = -1; dx <= 1; ++dx) {
                int64_t coords[3] = {center[0] + dx, center[1] + dy, center[2] + dz};
                uint32_t cell;
                if (!cell_index_from_coords(coords, cfg, &cell)) continue;
                uint64_t bin = batch * g->cell_count + cell;
                for (uint32_t s = g->bin_offsets[bin]; s < g->bin_offsets[bin + 1]; ++s) {
                    uint64_t j = base + g->permutation[s];
                    const float* pj = positions + 4 * j;
                    if (cfg->mode == NPA_MODE_PARTICLE) {
                        int64_t cj[3];
                        oracle_cell_coords(pj, cfg, cj);
                        if (cj[0] != coords[0] || cj[1] != coords[1] || cj[2] != coords[2]) continue;
                    }
                    float d[4];
                    neighbor_delta(pi, pj, cfg, d);
                    float r2 = d[0] * d[0];
                    for (uint32_t a = 1; a < cfg->dim; ++a) r2 += d[a] * d[a];
                    if (r2 < eps2) nbuf_push(out, (uint32_t)j, d, r2);
                }
            }
}

typedef struct hashgrid {
    uint32_t* bin_offsets;
    uint32_t* permutation;
    uint32_t* inverse;
    grid_view view;
} hashgrid;

static int hashgrid_build(const float* positions, uint32_t batch_size, uint32_t particle_count,
                          const npa_grid_cfg* cfg, hashgrid* h) {
    uint64_t total = (uint64_t)batch_size * particle_count;
    uint64_t bins = (uint64_t)batch_size * oracle_cell_count(cfg);
    h->bin_offsets = (uint32_t*)malloc((bins + 1) * sizeof(uint32_t));
    h->permutation = (uint32_t*)malloc((total ? total : 1) * sizeof(uint32_t));
    h->inverse = (uint32_t*)malloc((total ? total : 1) * sizeof(uint32_t));
    if (!h->bin_offsets || !h->permutation || !h->inverse) return NPA_ERR_OUT_OF_MEMORY;
    int st = oracle_build_hashgrid(positions, batch_size, particle_count, cfg, h->bin_offsets,
                                   h->permutation, h->inverse);
    h->view.bin_offsets = h->bin_offsets;
    h->view.permutation = h->permutation;
    h->view.particle_count = particle_count;
    h->view.cell_count = oracle_cell_count(cfg);
    return st;
}

static void hashgrid_free(hashgrid* h) {
    free(h->bin_offsets);
    free(h->permutation);
    free(h->inverse);
}

size_t oracle_neighbor_lists(const float* positions, uint32_t batch_size, uint32_t particle_count,
                             const npa_grid_cfg* cfg, uint32_t* offsets, uint32_t* indices) {
    if (oracle_grid_validate(cfg)) return (size_t)-1;
    hashgrid h;
    if (hashgrid_build(positions, batch_size, particle_count, cfg, &h)) {
        hashgrid_free(&h);
        return (size_t)-1;
    }
    uint64_t total = (uint64_t)batch_size * particle_count;
    nbuf buf = {0};
    size_t len = 0;
    offsets[0] = 0;
    for (uint64_t i = 0; i < total; ++i) {
        collect_neighbors(i, positions, &h.view, cfg, &buf);
        if (indices)
            for (size_t k = 0; k < buf.len; ++k) indices[len + k] = buf.v[k].j;
        len += buf.len;
        offsets[i + 1] = (uint32_t)len;
    }
    free(buf.v);
    hashgrid_free(&h);
    return len;
}

/* --------------------------------------------------------- SPH kernels */

/* smoothing_poly6_normalization / gradient_spiky_normalization
 * crates/burn_automata_kernels/src/reference/kernels.rs:126-140 */
static float poly6_norm(const npa_grid_cfg* cfg) {
    if (cfg->dim == 2) return 4.0f / (PI_F * powi_f32(cfg->eps, 8));
    return 315.0f / (64.0f * PI_F * powi_f32(cfg->eps, 9));
}
static float spiky_norm(const npa_grid_cfg* cfg) {
    if (cfg->dim == 2) return 10.0f / (PI_F * powi_f32(cfg->eps, 5));
    return 15.0f / (PI_F * powi_f32(cfg->eps, 6));
}

/* smoothing_poly6_kernel  kernels.rs:51-58 */
static float poly6(float r2, const npa_grid_cfg* cfg) {
    float eps2 = cfg->eps * cfg->eps;
    if (r2 >= eps2) return 0.0f;
    float x = eps2 - r2;
    return poly6_norm(cfg) * x * x * x;
}

/* spiky_gradient_kernel  kernels.rs:79-96 */
static void spiky_grad(const float delta[4], float r2, const npa_grid_cfg* cfg, float coeff,
                       float out[4]) {
    out[0] = out[1] = out[2] = out[3] = 0.0f;
    float eps2 = cfg->eps * cfg->eps;
    if (r2 <= 0.0f || r2 >= eps2) return;
    float r = sqrtf(r2);
    float t = cfg->eps - r;
    float mag = coeff * spiky_norm(cfg) * 3.0f * (t * t) / r;
    for (uint32_t a = 0; a < cfg->dim; ++a) out[a] = mag * delta[a];
}

/* RecipFinite::recip_finite  kernels.rs:146-154 */
static float recip_finite(float x) {
    if (fabsf(x) <= 1e-20f || !isfinite(x)) return 0.0f;
    return 1.0f / x;
}

/* safe_inverse_symmetric  kernels.rs:3-49 */
static void safe_inverse_symmetric(const float* m, uint32_t dim, float out[9]) {
    const float TOL = 1e-3f;
    for (int k = 0; k < 9; ++k) out[k] = 0.0f;
    if (dim == 2) {
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
        return;
    }
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

/* ------------------------------------------------------------- normalize */

/* log_normalize_vector  crates/burn_automata_kernels/src/reference/normalize.rs:60-69 */
static void log_normalize_vector(float* v, uint32_t n) {
    const float E = 1.0e-6f;
    float s = v[0] * v[0];
    for (uint32_t k = 1; k < n; ++k) s += v[k] * v[k];
    float norm = fmaxf(sqrtf(s + E * E), E);
    float scale = log1pf(norm) / norm;
    for (uint32_t k = 0; k < n; ++k) v[k] *= scale;
}

/* normalize_state_gradient  normalize.rs:5-30 */
static void normalize_state_gradient(float* grad, uint64_t total, uint32_t S,
                                     const npa_grid_cfg* cfg, const npa_perception_opts* o) {
    float eps0 = fmaxf(o->eps0, FLT_MIN);
    float scale = o->scale_equivariance ? cfg->eps / eps0 : 1.0f;
    const uint32_t d = cfg->dim;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)total; ++i) {
        float* pg = grad + (uint64_t)i * S * d;
        for (uint32_t c = 0; c < S; ++c) {
            for (uint32_t a = 0; a < d; ++a) pg[c * d + a] *= scale;
            if (o->log_norm_grad) log_normalize_vector(pg + c * d, d);
        }
    }
}

/* normalize_density_gradient  normalize.rs:32-58 */
static void normalize_density_gradient(float* grad, uint64_t total, uint32_t particle_count,
                                       const npa_grid_cfg* cfg, const npa_perception_opts* o) {
    float eps0 = fmaxf(o->eps0, FLT_MIN);
    float s1 = o->scale_equivariance ? powi_f32(cfg->eps / eps0, 1 + (int)cfg->dim) : 1.0f;
    float s2 = o->particle_density_equivariance
                   ? 1.0f / (float)(particle_count > 1 ? particle_count : 1)
                   : 1.0f;
    float scale = s1 * s2;
    const uint32_t d = cfg->dim;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)total; ++i) {
        float* pg = grad + (uint64_t)i * d;
        for (uint32_t a = 0; a < d; ++a) pg[a] *= scale;
        if (o->log_norm_density_grad) log_normalize_vector(pg, d);
    }
}

/* apply_moment_correction  normalize.rs:93-118 */
static void apply_moment_correction(float* grad, const float* moment, uint64_t total, uint32_t S,
                                    const npa_grid_cfg* cfg) {
    const uint32_t d = cfg->dim;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)total; ++i) {
        float* pg = grad + (uint64_t)i * S * d;
        float inv[9];
        safe_inverse_symmetric(moment + (uint64_t)i * d * d, d, inv);
        for (uint32_t c = 0; c < S; ++c) {
            float corrected[4];
            for (uint32_t o = 0; o < d; ++o) corrected[o] = 0.0f;
            for (uint32_t o = 0; o < d; ++o)
                for (uint32_t k = 0; k < d; ++k) corrected[o] += pg[c * d + k] * inv[k * d + o];
            for (uint32_t o = 0; o < d; ++o) pg[c * d + o] = corrected[o];
        }
    }
}

/* ------------------------------------------------------------ perception */

uint32_t oracle_feature_dims(uint32_t S, uint32_t dim, const npa_perception_opts* o) {
    /* forward.rs:100-103 */
    return S * 2 + (o->state_grad ? S * dim : 0) + (o->density_grad ? dim : 0) +
           (o->position_features ? dim : 0);
}

/* density  forward.rs:145-160 */
/* Every pass below runs over `rows` targets: particle sel[r] (or r when sel is NULL) writes
 * output row r, so a pass can evaluate a sample of a system too large for a full pass. */
static void pass_density(const float* positions, const grid_view* g, const npa_grid_cfg* cfg,
                         const uint32_t* sel, uint64_t rows, float* rho_out) {
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(i, positions, g, cfg, &buf);
            float rho = 0.0f;
            for (size_t k = 0; k < buf.len; ++k) rho += poly6(buf.v[k].r2, cfg);
            rho_out[r] = rho;
        }
        free(buf.v);
    }
}

/* second_pass_particle  forward.rs:248-295 (density_grad && state_grad branch) */
static void pass_second(const float* positions, const float* states, const float* density,
                        uint32_t S, const grid_view* g, const npa_grid_cfg* cfg, const uint32_t* sel,
                        uint64_t rows, float* blur, float* sgrad, float* dgrad, float* moment) {
    const uint32_t d = cfg->dim;
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t idx = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(idx, positions, g, cfg, &buf);
            float* blur_row = blur + (uint64_t)r * S;
            float* grad_row = sgrad + (uint64_t)r * S * d;
            float* dg_row = dgrad + (uint64_t)r * d;
            float* m_row = moment ? moment + (uint64_t)r * d * d : NULL;
            const float* si = states + idx * S;
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                float volume_j = recip_finite(density[n->j]);
                float smooth = poly6(n->r2, cfg);
                const float* sj = states + (uint64_t)n->j * S;
                for (uint32_t c = 0; c < S; ++c) blur_row[c] += sj[c] * smooth * volume_j;
                if (idx == n->j) continue;
                float dgk[4], vg[4];
                spiky_grad(n->delta, n->r2, cfg, 1.0f, dgk);
                for (uint32_t a = 0; a < d; ++a) dg_row[a] += dgk[a];
                spiky_grad(n->delta, n->r2, cfg, volume_j, vg);
                for (uint32_t c = 0; c < S; ++c) {
                    float diff = sj[c] - si[c];
                    for (uint32_t a = 0; a < d; ++a) grad_row[c * d + a] += diff * vg[a];
                }
                if (m_row)
                    for (uint32_t r = 0; r < d; ++r)
                        for (uint32_t c = 0; c < d; ++c) m_row[r * d + c] += n->delta[r] * vg[c];
            }
        }
        free(buf.v);
    }
}

/* blur_state  forward.rs:162-184 */
static void pass_blur(const float* positions, const float* states, const float* density,
                      uint32_t S, const grid_view* g, const npa_grid_cfg* cfg, const uint32_t* sel,
                      uint64_t rows, float* out) {
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(i, positions, g, cfg, &buf);
            float* dst = out + (uint64_t)r * S;
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                float volume_j = recip_finite(density[n->j]);
                float w = poly6(n->r2, cfg) * volume_j;
                const float* sj = states + (uint64_t)n->j * S;
                for (uint32_t c = 0; c < S; ++c) dst[c] += sj[c] * w;
            }
        }
        free(buf.v);
    }
}

/* moment_matrix  forward.rs:357-382 */
static void pass_moment(const float* positions, const float* density, const grid_view* g,
                        const npa_grid_cfg* cfg, const uint32_t* sel, uint64_t rows, float* out) {
    const uint32_t d = cfg->dim;
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(i, positions, g, cfg, &buf);
            float* dst = out + (uint64_t)r * d * d;
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (i == n->j) continue;
                float volume_j = recip_finite(density[n->j]);
                float grad[4];
                spiky_grad(n->delta, n->r2, cfg, volume_j, grad);
                for (uint32_t r = 0; r < d; ++r)
                    for (uint32_t c = 0; c < d; ++c) dst[r * d + c] += n->delta[r] * grad[c];
            }
        }
        free(buf.v);
    }
}

/* compute_state_gradient  forward.rs:297-333 */
static void pass_state_gradient(const float* positions, const float* states,
                                const float* density, uint32_t S, const grid_view* g,
                                const npa_grid_cfg* cfg, const uint32_t* sel, uint64_t rows, int hybrid,
                                float* out) {
    const uint32_t d = cfg->dim;
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(i, positions, g, cfg, &buf);
            float* dst = out + (uint64_t)r * S * d;
            const float* si = states + i * S;
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (i == n->j) continue;
                float volume_j = recip_finite(density[n->j]);
                float grad[4];
                spiky_grad(n->delta, n->r2, cfg, volume_j, grad);
                const float* sj = states + (uint64_t)n->j * S;
                for (uint32_t c = 0; c < S; ++c) {
                    float diff = sj[c] - si[c];
                    for (uint32_t a = 0; a < d; ++a) dst[c * d + a] += diff * grad[a];
                }
            }
        }
        free(buf.v);
    }
    if (hybrid) {
        float* moment = (float*)calloc(rows * d * d + 1, sizeof(float));
        pass_moment(positions, density, g, cfg, sel, rows, moment);
        apply_moment_correction(out, moment, rows, S, cfg);
        free(moment);
    }
}

/* compute_density_gradient  forward.rs:335-355 */
static void pass_density_gradient(const float* positions, const grid_view* g,
                                  const npa_grid_cfg* cfg, const uint32_t* sel, uint64_t rows, float* out) {
    const uint32_t d = cfg->dim;
#pragma omp parallel
    {
        nbuf buf = {0};
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            collect_neighbors(i, positions, g, cfg, &buf);
            float* dst = out + (uint64_t)r * d;
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (i == n->j) continue;
                float grad[4];
                spiky_grad(n->delta, n->r2, cfg, 1.0f, grad);
                for (uint32_t a = 0; a < d; ++a) dst[a] += grad[a];
            }
        }
        free(buf.v);
    }
}

/* The second half of perceive_with_options (forward.rs:26-143) for targets sel[0..rows) (all
 * particles when sel is NULL), given the density of every particle: second pass, moment
 * correction, normalisation and feature rows, written to rows 0..rows of the outputs. */
static int perceive_rows(const float* positions, const float* states, uint32_t particle_count,
                         uint32_t S, const npa_grid_cfg* cfg, const npa_perception_opts* o,
                         const grid_view* g, const float* density, const uint32_t* sel,
                         uint64_t rows, float* features, float* blurred_out, float* sgrad_out,
                         float* dgrad_out) {
    const uint32_t d = cfg->dim;
    float* blur = (float*)calloc(rows * S + 1, sizeof(float));
    float* sgrad = (float*)calloc(o->state_grad ? rows * S * d + 1 : 1, sizeof(float));
    float* dgrad = (float*)calloc(o->density_grad ? rows * d + 1 : 1, sizeof(float));
    if (!blur || !sgrad || !dgrad) {
        free(blur);
        free(sgrad);
        free(dgrad);
        return NPA_ERR_OUT_OF_MEMORY;
    }
    if (o->state_grad && o->density_grad) {
        float* moment = o->hybrid_state_gradient ? (float*)calloc(rows * d * d + 1, sizeof(float)) : NULL;
        pass_second(positions, states, density, S, g, cfg, sel, rows, blur, sgrad, dgrad, moment);
        if (moment) apply_moment_correction(sgrad, moment, rows, S, cfg);
        normalize_state_gradient(sgrad, rows, S, cfg, o);
        normalize_density_gradient(dgrad, rows, particle_count, cfg, o);
        free(moment);
    } else {
        pass_blur(positions, states, density, S, g, cfg, sel, rows, blur);
        if (o->state_grad) {
            pass_state_gradient(positions, states, density, S, g, cfg, sel, rows,
                                (int)o->hybrid_state_gradient, sgrad);
            normalize_state_gradient(sgrad, rows, S, cfg, o);
        }
        if (o->density_grad) {
            pass_density_gradient(positions, g, cfg, sel, rows, dgrad);
            normalize_density_gradient(dgrad, rows, particle_count, cfg, o);
        }
    }

    const uint32_t F = oracle_feature_dims(S, d, o);
    if (features) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const uint64_t i = sel ? sel[r] : (uint64_t)r;
            float* f = features + (uint64_t)r * F;
            uint32_t cur = 0;
            memcpy(f + cur, states + i * S, S * sizeof(float));
            cur += S;
            memcpy(f + cur, blur + (uint64_t)r * S, S * sizeof(float));
            cur += S;
            if (o->state_grad) {
                memcpy(f + cur, sgrad + (uint64_t)r * S * d, S * d * sizeof(float));
                cur += S * d;
            }
            if (o->density_grad) {
                memcpy(f + cur, dgrad + (uint64_t)r * d, d * sizeof(float));
                cur += d;
            }
            if (o->position_features) memcpy(f + cur, positions + 4 * i, d * sizeof(float));
        }
    }
    if (blurred_out) memcpy(blurred_out, blur, rows * S * sizeof(float));
    if (sgrad_out && o->state_grad) memcpy(sgrad_out, sgrad, rows * S * d * sizeof(float));
    if (dgrad_out && o->density_grad) memcpy(dgrad_out, dgrad, rows * d * sizeof(float));
    free(blur);
    free(sgrad);
    free(dgrad);
    return NPA_OK;
}

/* perceive_with_options  crates/burn_automata_kernels/src/reference/forward.rs:26-143 */
int oracle_perceive(const float* positions, const float* states, uint32_t batch_size,
                    uint32_t particle_count, uint32_t S, const npa_grid_cfg* cfg,
                    const npa_perception_opts* o, float* features, float* density,
                    float* blurred_out, float* sgrad_out, float* dgrad_out) {
    int st = oracle_grid_validate(cfg);
    if (st) return st;
    const uint64_t total = (uint64_t)batch_size * particle_count;
    hashgrid h;
    st = hashgrid_build(positions, batch_size, particle_count, cfg, &h);
    if (st) {
        hashgrid_free(&h);
        return st;
    }
    pass_density(positions, &h.view, cfg, NULL, total, density);
    st = perceive_rows(positions, states, particle_count, S, cfg, o, &h.view, density, NULL, total,
                       features, blurred_out, sgrad_out, dgrad_out);
    hashgrid_free(&h);
    return st;
}

/* density (forward.rs:145-160) of the particles sel[0..rows) only, into rho_out[0..rows). */
int oracle_density_rows(const float* positions, uint32_t batch_size, uint32_t particle_count,
                        const npa_grid_cfg* cfg, const uint32_t* sel, uint64_t rows, float* rho_out) {
    int st = oracle_grid_validate(cfg);
    if (st) return st;
    hashgrid h;
    st = hashgrid_build(positions, batch_size, particle_count, cfg, &h);
    if (!st) pass_density(positions, &h.view, cfg, sel, rows, rho_out);
    hashgrid_free(&h);
    return st;
}

/* ------------------------------------------------------------------ model */

/* NpaConfig::scale_equivariant / particle_density_equivariant  config.rs:145-154 and the
 * PerceptionOptions that step_cpu builds  crates/burn_automata/src/model.rs:784-800 */
void oracle_perception_opts_for_model(const npa_model_cfg* m, npa_perception_opts* o) {
    o->state_grad = m->state_grad;
    o->density_grad = m->density_grad;
    o->eps0 = m->eps0;
    o->scale_equivariance = m->equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE;
    o->particle_density_equivariance = m->equivariance == NPA_EQUIV_PARTICLE_DENSITY ||
                                       m->equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE;
    o->log_norm_grad = m->log_norm_grad;
    o->log_norm_density_grad = m->log_norm_density_grad;
    o->hybrid_state_gradient = 1;
    o->position_features = m->position_features;
}

/* NpaConfig::perception_dims  crates/burn_automata/src/config.rs:133-139 (no auxiliary inputs) */
uint32_t oracle_model_perception_dims(const npa_model_cfg* m) {
    return m->state_dims * 2 + (m->state_grad ? m->state_dims * m->spatial_dims : 0) +
           (m->density_grad ? m->spatial_dims : 0) + (m->position_features ? m->spatial_dims : 0);
}

/* forward_update_from_features  crates/burn_automata/src/model.rs:900-940 */
int oracle_forward_update(const float* features, uint32_t rows, const npa_model_cfg* m,
                          const npa_weights* w, float* update) {
    const uint32_t F = oracle_model_perception_dims(m), H = m->hidden_dims;
    const uint32_t O = m->spatial_dims + m->state_dims;
#pragma omp parallel
    {
        float* hidden = (float*)malloc((H ? H : 1) * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < (int64_t)rows; ++r) {
            const float* f = features + (uint64_t)r * F;
            for (uint32_t h = 0; h < H; ++h) {
                float sum = w->b1[h];
                const float* wr = w->w1 + (uint64_t)h * F;
                for (uint32_t i = 0; i < F; ++i) sum += wr[i] * f[i];
                hidden[h] = fmaxf(sum, 0.0f);
            }
            float* u = update + (uint64_t)r * O;
            for (uint32_t o = 0; o < O; ++o) {
                float sum = w->b2[o];
                const float* wr = w->w2 + (uint64_t)o * H;
                for (uint32_t h = 0; h < H; ++h) sum += wr[h] * hidden[h];
                u[o] = sum;
            }
        }
        free(hidden);
    }
    return NPA_OK;
}

/* NpaConfig::motion_eps  config.rs:156-162 */
static float motion_eps(const npa_model_cfg* m, float grid_eps) {
    return m->equivariance == NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE ? grid_eps : m->eps0;
}

/* forward_from_features_with_eps  model.rs:867-898 */
int oracle_forward_from_features(const float* features, uint32_t rows, const npa_model_cfg* m,
                                 const npa_weights* w, float eps, float* dx, float* ds) {
    const uint32_t O = m->spatial_dims + m->state_dims, S = m->state_dims, d = m->spatial_dims;
    float* update = (float*)malloc(((uint64_t)rows * O + 1) * sizeof(float));
    if (!update) return NPA_ERR_OUT_OF_MEMORY;
    oracle_forward_update(features, rows, m, w, update);
    const float meps = motion_eps(m, eps);
    for (uint64_t r = 0; r < rows; ++r) {
        const float* u = update + r * O;
        float norm = 0.0f;
        for (uint32_t a = 0; a < d; ++a) norm += u[a] * u[a];
        norm = sqrtf(norm);
        float* px = dx + 4 * r;
        px[0] = px[1] = px[2] = px[3] = 0.0f;
        for (uint32_t a = 0; a < d; ++a) px[a] = m->alpha * u[a] * meps / (1.0f + norm);
        memcpy(ds + r * S, u + d, S * sizeof(float));
    }
    free(update);
    return NPA_OK;
}

/* euler_step  crates/burn_automata_kernels/src/reference/step.rs:4-55 */
int oracle_euler_step(const float* positions, const float* states, const float* dx,
                      const float* ds, uint32_t batch_size, uint32_t particle_count, uint32_t S,
                      const npa_grid_cfg* cfg, float dt, const float* mask, float* out_pos,
                      float* out_states) {
    const uint64_t total = (uint64_t)batch_size * particle_count;
    const int mem = spatial_mem_dims(cfg);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)total; ++i) {
        float m = mask ? mask[i] : 1.0f;
        float p[4];
        memcpy(p, positions + 4 * (uint64_t)i, sizeof(p));
        for (int a = 0; a < mem; ++a) p[a] += dt * dx[4 * (uint64_t)i + a] * m;
        /* wrap_position  crates/burn_automata_kernels/src/hashgrid.rs:183-193 */
        if (cfg->boundary == NPA_BOUNDARY_PERIODIC) {
            for (uint32_t a = 0; a < cfg->dim; ++a) {
                float extent = (float)cfg->grid_size[a] * cfg->eps;
                float half = extent * 0.5f;
                p[a] = rem_euclid_f32(p[a] + half, extent) - half;
            }
        }
        memcpy(out_pos + 4 * (uint64_t)i, p, sizeof(p));
        const float* s = states + (uint64_t)i * S;
        const float* dsr = ds + (uint64_t)i * S;
        float* os = out_states + (uint64_t)i * S;
        for (uint32_t c = 0; c < S; ++c) {
            float next = s[c] + dt * dsr[c] * m;
            if (cfg->dim == 3 && S > 3 && (c == 3 || (S > 8 && c == 8)))
                next = clamp_f32(next, -8.0f, 24.0f); /* GROWTH_3D_{MIN,MAX}_OPACITY_LOGIT types.rs:1-2 */
            os[c] = next;
        }
    }
    return NPA_OK;
}

/* position_conditioned_3d_maturity_gate / motion_gate  crates/burn_automata/src/rollout/mod.rs:67-91 */
static float maturity_gate(float liveness) { return clamp_f32((4.0f - liveness) * 2.0f, 0.0f, 1.0f); }
static float motion_gate(float liveness, float signed_distance, int anchored) {
    if (anchored) return 0.0f;
    float state_gate = maturity_gate(liveness);
    float distance_gate = clamp_f32((fabsf(signed_distance) - 0.01f) / 0.02f, 0.0f, 1.0f);
    return state_gate * distance_gate;
}

/* The update half of NpaModel::step_cpu (model.rs:800-858) for `rows` feature rows: the MLP and
 * motion scaling, the 3D gates and the masked Euler step. Row r is particle sel[r] (r when sel is
 * NULL) of `positions` / `states` / `mask`; outputs are written to rows 0..rows. */
static int update_rows(const float* positions, const float* states, const float* mask,
                       const uint32_t* sel, uint64_t rows, const npa_grid_cfg* grid,
                       const npa_model_cfg* m, const npa_weights* w, float dt,
                       const float* features, float* out_pos, float* out_states, float* out_dx,
                       float* out_ds) {
    const uint32_t S = m->state_dims;
    float* dx = (float*)malloc((rows * 4 + 1) * sizeof(float));
    float* ds = (float*)malloc((rows * S + 1) * sizeof(float));
    float* gp = sel ? (float*)malloc((rows * 4 + 1) * sizeof(float)) : NULL;
    float* gs = sel ? (float*)malloc((rows * S + 1) * sizeof(float)) : NULL;
    float* gm = sel && mask ? (float*)malloc((rows + 1) * sizeof(float)) : NULL;
    int st = (!dx || !ds || (sel && (!gp || !gs)) || (sel && mask && !gm)) ? NPA_ERR_OUT_OF_MEMORY : NPA_OK;
    if (!st && sel) {
        for (uint64_t r = 0; r < rows; ++r) {
            memcpy(gp + 4 * r, positions + 4 * (uint64_t)sel[r], 4 * sizeof(float));
            memcpy(gs + r * S, states + (uint64_t)sel[r] * S, S * sizeof(float));
            if (gm) gm[r] = mask[sel[r]];
        }
        positions = gp;
        states = gs;
        mask = gm;
    }
    if (!st) st = oracle_forward_from_features(features, (uint32_t)rows, m, w, grid->eps, dx, ds);
    if (!st && m->spatial_dims == 3 && m->position_features && S > 3) {
        for (uint64_t r = 0; r < rows; ++r) {
            const float* s = states + r * S;
            float liveness = s[3];                    /* GROWTH_3D_LIVENESS_CHANNEL */
            float signed_distance = s[7];             /* UV_TORUS_SIGNED_DISTANCE_STATE_OFFSET */
            float sg = maturity_gate(liveness);
            float mg = motion_gate(liveness, signed_distance, positions[4 * r + 3] >= 0.5f);
            for (uint32_t a = 0; a < m->spatial_dims; ++a) dx[4 * r + a] *= mg;
            for (uint32_t c = 0; c < S; ++c) ds[r * S + c] *= sg;
        }
    }
    if (!st) st = oracle_euler_step(positions, states, dx, ds, 1, (uint32_t)rows, S, grid, dt, mask,
                                    out_pos, out_states);
    if (!st && out_dx) memcpy(out_dx, dx, rows * 4 * sizeof(float));
    if (!st && out_ds) memcpy(out_ds, ds, rows * S * sizeof(float));
    free(dx);
    free(ds);
    free(gp);
    free(gs);
    free(gm);
    return st;
}

/* NpaModel::step_cpu  crates/burn_automata/src/model.rs:768-858 */
int oracle_step(const float* positions, const float* states, uint32_t batch_size,
                uint32_t particle_count, const npa_grid_cfg* grid, const npa_model_cfg* m,
                const npa_weights* w, float dt, const float* mask, float* out_pos,
                float* out_states, float* out_density, float* out_dx, float* out_ds) {
    if (!(m->spatial_dims == 2 || m->spatial_dims == 3)) return NPA_ERR_INVALID_MODEL;
    if (grid->dim != m->spatial_dims) return NPA_ERR_INVALID_ARGUMENT;
    const uint64_t total = (uint64_t)batch_size * particle_count;
    const uint32_t S = m->state_dims;
    npa_perception_opts o;
    oracle_perception_opts_for_model(m, &o);
    const uint32_t F = oracle_model_perception_dims(m);
    float* features = (float*)malloc((total * F + 1) * sizeof(float));
    float* density = (float*)malloc((total + 1) * sizeof(float));
    float* blur = (float*)malloc((total * S + 1) * sizeof(float));
    if (!features || !density || !blur) {
        free(features);
        free(density);
        free(blur);
        return NPA_ERR_OUT_OF_MEMORY;
    }

    double t0 = omp_get_wtime();
    int st = oracle_perceive(positions, states, batch_size, particle_count, S, grid, &o, features,
                             density, blur, NULL, NULL);
    double t1 = omp_get_wtime();
    if (!st) st = update_rows(positions, states, mask, NULL, total, grid, m, w, dt, features, out_pos,
                              out_states, out_dx, out_ds);
    double t2 = omp_get_wtime();
    g_phase_perceive = t1 - t0;
    g_phase_mlp = t2 - t1;  /* MLP, gates and Euler */
    g_phase_integrate = 0.0;
    if (out_density) memcpy(out_density, density, total * sizeof(float));
    free(features);
    free(density);
    free(blur);
    return st;
}

/* NpaModel::step_cpu for the particles sel[0..rows) only, given the density of every particle
 * (the first pass's output): second pass, feature rows, update MLP, gates and Euler step of those
 * particles, written to rows 0..rows of out_positions / out_states. */
int oracle_step_rows(const float* positions, const float* states, uint32_t batch_size,
                     uint32_t particle_count, const npa_grid_cfg* grid, const npa_model_cfg* m,
                     const npa_weights* w, float dt, const float* mask, const float* density,
                     const uint32_t* sel, uint64_t rows, float* out_pos, float* out_states) {
    if (!(m->spatial_dims == 2 || m->spatial_dims == 3)) return NPA_ERR_INVALID_MODEL;
    if (grid->dim != m->spatial_dims) return NPA_ERR_INVALID_ARGUMENT;
    int st = oracle_grid_validate(grid);
    if (st) return st;
    npa_perception_opts o;
    oracle_perception_opts_for_model(m, &o);
    const uint32_t F = oracle_model_perception_dims(m);
    float* features = (float*)malloc((rows * F + 1) * sizeof(float));
    if (!features) return NPA_ERR_OUT_OF_MEMORY;
    hashgrid h;
    st = hashgrid_build(positions, batch_size, particle_count, grid, &h);
    if (!st) st = perceive_rows(positions, states, particle_count, m->state_dims, grid, &o, &h.view,
                                density, sel, rows, features, NULL, NULL, NULL);
    if (!st) st = update_rows(positions, states, mask, sel, rows, grid, m, w, dt, features, out_pos,
                              out_states, NULL, NULL);
    hashgrid_free(&h);
    free(features);
    return st;
}

/* ------------------------------------------------------------------- mask */

/* hash_u32 / random01  crates/burn_automata/src/gpu_step.wgsl:1019-1031 */
uint32_t oracle_hash_u32(uint32_t x) {
    x = (x ^ 61u) ^ (x >> 16);
    x = x + (x << 3);
    x = x ^ (x >> 4);
    x = x * 0x27d4eb2du;
    x = x ^ (x >> 15);
    return x;
}

float oracle_random01(uint32_t particle, uint32_t step, uint32_t seed) {
    uint32_t mixed = oracle_hash_u32(particle ^ oracle_hash_u32(step + 0x9e3779b9u) ^ seed);
    return (float)(mixed >> 8) * (1.0f / 16777216.0f);
}

/* gpu_random_seed  crates/burn_automata/src/gpu/helpers/params.rs:186-188 */
uint32_t oracle_gpu_random_seed(uint64_t seed) { return (uint32_t)seed ^ (uint32_t)(seed >> 32); }

/* update_mask  gpu_step.wgsl:1033-1056, lane seeds gpu_lane_seeds
 * crates/burn_automata/src/gpu/executor/state.rs:1282-1315 (shared seed, no per-lane seeds) */
void oracle_update_mask(uint32_t batch_size, uint32_t particle_count, float p, uint32_t step,
                        uint64_t seed, float* mask) {
    const uint32_t base = oracle_gpu_random_seed(seed);
    for (uint64_t b = 0; b < batch_size; ++b) {
        uint32_t lane_seed = base ^ (uint32_t)(b * particle_count);
        for (uint64_t i = 0; i < particle_count; ++i) {
            float v;
            if (p >= 1.0f) v = 1.0f;
            else if (p <= 0.0f) v = 0.0f;
            else v = oracle_random01((uint32_t)i, step, lane_seed) < p ? 1.0f : 0.0f;
            mask[b * particle_count + i] = v;
        }
    }
}

/* run_rollout_from_particles_with_mask_schedule  crates/burn_automata/src/rollout/mod.rs:240-297,
 * with the device mask schedule in place of the host StdRng stream. */
int oracle_rollout(float* positions, float* states, uint32_t batch_size, uint32_t particle_count,
                   const npa_grid_cfg* grid, const npa_model_cfg* m, const npa_weights* w,
                   float dt, float update_prob, uint64_t seed, uint32_t start_step,
                   uint32_t steps) {
    const uint64_t total = (uint64_t)batch_size * particle_count;
    const uint32_t S = m->state_dims;
    float* mask = (float*)malloc((total + 1) * sizeof(float));
    float* np = (float*)malloc((total * 4 + 1) * sizeof(float));
    float* ns = (float*)malloc((total * S + 1) * sizeof(float));
    if (!mask || !np || !ns) return NPA_ERR_OUT_OF_MEMORY;
    double acc[3] = {0, 0, 0};
    int st = NPA_OK;
    for (uint32_t k = 0; k < steps && !st; ++k) {
        oracle_update_mask(batch_size, particle_count, update_prob, start_step + k, seed, mask);
        st = oracle_step(positions, states, batch_size, particle_count, grid, m, w, dt, mask, np, ns,
                         NULL, NULL, NULL);
        memcpy(positions, np, total * 4 * sizeof(float));
        memcpy(states, ns, total * S * sizeof(float));
        acc[0] += g_phase_perceive;
        acc[1] += g_phase_mlp;
        acc[2] += g_phase_integrate;
    }
    g_phase_perceive = acc[0];
    g_phase_mlp = acc[1];
    g_phase_integrate = acc[2];
    free(mask);
    free(np);
    free(ns);
    return st;
}

/* ------------------------------------------------------------------ decode */

/* decode_sh_coeffs  crates/burn_automata_kernels/src/gaussian.rs:127-132 */
uint32_t oracle_decode_sh_coeffs(const npa_gaussian_decode_cfg* cfg) {
    if (cfg->mode == NPA_DECODE_SH0_ORIENTED) return (cfg->sh_degree + 1) * (cfg->sh_degree + 1);
    return 1;
}

static float sigmoid_f32(float v) { return 1.0f / (1.0f + expf(-v)); } /* gaussian.rs:210-212 */

/* decode_gaussians_3d  gaussian.rs:53-100 (+ validate_decode_layout 102-125,
 * decode_sh 134-158, decode_scale_opacity 160-208, normalize_quat 214-223).
 * Returns NPA_ERR_INVALID_ARGUMENT where the reference panics. */
int oracle_decode_gaussians_3d(const float* positions, const float* states, uint32_t count,
                               uint32_t S, const npa_gaussian_decode_cfg* cfg, float* pos_vis,
                               float* sh, float* rotation, float* scale_opacity) {
    const uint32_t K = oracle_decode_sh_coeffs(cfg);
    switch (cfg->mode) {
        case NPA_DECODE_PARTICLE_POINT:
        case NPA_DECODE_SH0_FIXED_SCALE:
            if (S < 3) return NPA_ERR_INVALID_ARGUMENT;
            break;
        case NPA_DECODE_SH0_LEARNED_SCALE:
            if (S < 5) return NPA_ERR_INVALID_ARGUMENT;
            break;
        case NPA_DECODE_SH0_ORIENTED:
            if (S < K * 3 + 8) return NPA_ERR_INVALID_ARGUMENT;
            break;
        default:
            return NPA_ERR_INVALID_ARGUMENT;
    }
    for (uint64_t idx = 0; idx < count; ++idx) {
        const float* s = states + idx * S;
        const float* p = positions + 4 * idx;
        uint32_t color_start = cfg->mode == NPA_DECODE_SH0_ORIENTED ? S - K * 3 : S - 3;
        for (uint32_t k = 0; k < K; ++k) {
            uint32_t base = color_start + k * 3;
            for (int ch = 0; ch < 3; ++ch)
                sh[(idx * K + k) * 3 + ch] = clamp_f32(s[base + ch] + 0.5f, 0.0f, 1.0f);
        }
        float* rot = rotation + 4 * idx;
        if (cfg->mode == NPA_DECODE_SH0_ORIENTED) {
            uint32_t rs = color_start - 4;
            float q[4] = {s[rs], s[rs + 1], s[rs + 2], s[rs + 3]};
            float norm = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
            if (norm <= 1e-8f) {
                q[0] = 1.0f;
                q[1] = q[2] = q[3] = 0.0f;
            } else {
                for (int k = 0; k < 4; ++k) q[k] /= norm;
            }
            memcpy(rot, q, sizeof(q));
        } else {
            rot[0] = 1.0f;
            rot[1] = rot[2] = rot[3] = 0.0f;
        }
        float* so = scale_opacity + 4 * idx;
        switch (cfg->mode) {
            case NPA_DECODE_PARTICLE_POINT: {
                float sc = fmaxf(cfg->min_scale, 1.0e-6f);
                so[0] = so[1] = so[2] = sc;
                so[3] = 1.0f;
            } break;
            case NPA_DECODE_SH0_FIXED_SCALE: {
                float sc = clamp_f32(cfg->sigma, cfg->min_scale, cfg->max_scale);
                so[0] = so[1] = so[2] = sc;
                so[3] = clamp_f32(cfg->opacity_scale, cfg->min_opacity, cfg->max_opacity);
            } break;
            case NPA_DECODE_SH0_LEARNED_SCALE: {
                float scale_logit = clamp_f32(s[S - 5], -8.0f, 8.0f);
                float opacity_logit = clamp_f32(s[S - 4], -12.0f, 12.0f);
                float sc = clamp_f32(cfg->sigma * expf(scale_logit), cfg->min_scale, cfg->max_scale);
                float op = clamp_f32(sigmoid_f32(opacity_logit), cfg->min_opacity, cfg->max_opacity) *
                           cfg->opacity_scale;
                so[0] = so[1] = so[2] = sc;
                so[3] = clamp_f32(op, cfg->min_opacity, cfg->max_opacity);
            } break;
            default: { /* oriented */
                uint32_t anis = color_start - 4 - 4;
                float ma = fmaxf(cfg->max_anisotropy, 1e-6f);
                float ax = tanhf(s[anis] / ma) * cfg->max_anisotropy;
                float ay = tanhf(s[anis + 1] / ma) * cfg->max_anisotropy;
                float az = tanhf(s[anis + 2] / ma) * cfg->max_anisotropy;
                float ol = tanhf(s[anis + 3] / ma) * cfg->max_anisotropy;
                so[0] = clamp_f32(cfg->sigma * expf(ax), cfg->min_scale, cfg->max_scale);
                so[1] = clamp_f32(cfg->sigma * expf(ay), cfg->min_scale, cfg->max_scale);
                so[2] = clamp_f32(cfg->sigma * expf(az), cfg->min_scale, cfg->max_scale);
                so[3] = clamp_f32(cfg->opacity_scale * expf(ol), cfg->min_opacity, cfg->max_opacity);
            } break;
        }
        float* pv = pos_vis + 4 * idx;
        pv[0] = p[0];
        pv[1] = p[1];
        pv[2] = p[2];
        pv[3] = 1.0f;
    }
    return NPA_OK;
}

/* write_gaussian_from_output  crates/burn_automata/src/gpu_step.wgsl:4963-5052: the executor's
 * planar export for the viewer (write_gaussian_main 4929-4936), per particle of a state's current
 * buffers. SH colour write_gaussian_sh0_color 4981-4990 (48 coefficients, only the DC triple
 * non-zero), geometry write_gaussian_geometry_from_output 4992-5052, channel helpers
 * output_state_channel / output_tail_state_channel / output_material_opacity_logit 1565-1591,
 * sigmoid 1561-1563. particle_count is the per-system N (params.rs:142). The material branch
 * (material_gaussian_geometry) belongs to the adaptive rollouts and is not restated. normalize()
 * is evaluated as v / sqrt(v.x^2 + v.y^2 + v.z^2 + v.w^2) and length() as sqrt(x^2 + y^2 + z^2),
 * in that order. */
#define ORACLE_SH_COEFFS 48u
static const float ORACLE_SH_C0 = 0.28209479177387814f;

static float export_channel(const float* s, uint32_t S, uint32_t c) { /* output_state_channel */
    if (c < S) return s[c];
    return S > 0 ? s[0] : 0.0f;
}

static float export_tail_channel(const float* s, uint32_t S, uint32_t off) { /* output_tail_state_channel */
    return S > off ? export_channel(s, S, S - 1 - off) : export_channel(s, S, 0);
}

int oracle_write_gaussians(const float* positions, const float* states, uint64_t total, uint32_t particle_count,
                           uint32_t S, uint32_t dim, float eps, int position_features, float* pos_vis, float* sh,
                           float* rotation, float* scale_opacity) {
    if (dim != 2 && dim != 3) return NPA_ERR_INVALID_DIM;
    const int normal_branch = dim == 3 && position_features && S >= 9;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)total; ++i) {
        const uint64_t idx = (uint64_t)i;
        const float* p = positions + 4 * idx;
        const float* s = states + idx * S;
        float* pv = pos_vis + 4 * idx;
        pv[0] = p[0];
        pv[1] = p[1];
        pv[2] = dim == 3 ? p[2] : 0.0f;
        pv[3] = 1.0f;
        const float tail[3] = {export_tail_channel(s, S, 2), export_tail_channel(s, S, 1),
                               export_tail_channel(s, S, 0)};
        float* c = sh + idx * ORACLE_SH_COEFFS;
        for (uint32_t k = 0; k < ORACLE_SH_COEFFS; ++k) c[k] = 0.0f;
        for (int ch = 0; ch < 3; ++ch) {
            const float color = clamp_f32(tail[ch] + 0.5f, 0.0f, 1.0f);
            c[ch] = (color - 0.5f) / ORACLE_SH_C0;
        }
        float scale[3], rot[4] = {1.0f, 0.0f, 0.0f, 0.0f};
        const float iso = fmaxf(eps * 0.12f, 0.00008f);
        scale[0] = scale[1] = scale[2] = iso;
        if (normal_branch) {
            const float n[3] = {export_channel(s, S, 4), export_channel(s, S, 5), export_channel(s, S, 6)};
            const float nn = sqrtf(n[0] * n[0] + n[1] * n[1] + n[2] * n[2]);
            float u[3] = {0.0f, 0.0f, 1.0f};
            if (nn > 1.0e-6f && nn < 1.0e20f) {
                u[0] = n[0] / nn;
                u[1] = n[1] / nn;
                u[2] = n[2] / nn;
            }
            if (u[2] <= -0.999999f) {
                rot[0] = 0.0f;
                rot[1] = 1.0f;
                rot[2] = 0.0f;
                rot[3] = 0.0f;
            } else {
                const float q[4] = {1.0f + u[2], -u[1], u[0], 0.0f};
                const float ql = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
                for (int k = 0; k < 4; ++k) rot[k] = q[k] / ql;
            }
            const float density_scale =
                clamp_f32(sqrtf(4096.0f / fmaxf((float)particle_count, 1.0f)), 0.4f, 2.0f);
            const float tangent =
                fmaxf(clamp_f32(eps * 0.32f * density_scale, eps * 0.08f, eps * 0.64f), 0.00008f);
            scale[0] = tangent;
            scale[1] = tangent;
            scale[2] = fmaxf(tangent * 0.18f, 0.00008f);
        }
        float opacity = 1.0f;
        if (dim == 3) {
            const float logit = export_channel(s, S, S > 8 ? 8u : 3u);
            opacity = clamp_f32(1.0f / (1.0f + expf(-logit)), 0.001f, 0.95f);
        }
        float* r = rotation + 4 * idx;
        for (int k = 0; k < 4; ++k) r[k] = rot[k];
        float* so = scale_opacity + 4 * idx;
        so[0] = scale[0];
        so[1] = scale[1];
        so[2] = scale[2];
        so[3] = opacity * 1.0f;
    }
    return NPA_OK;
}

/* splat_particles_2d  crates/burn_automata_kernels/src/splat.rs:30-93 */
int oracle_splat_particles_2d(const float* positions, const float* colors, uint32_t count,
                              const npa_splat2d_cfg* cfg, float* image) {
    const int64_t size = cfg->image_size;
    memset(image, 0, (size_t)(size * size * 4) * sizeof(float));
    float sigma = cfg->sigma;
    if (cfg->normalize_color) sigma = sigma * (float)size * cfg->pixel_size / (cfg->hi - cfg->lo);
    float rf = fmaxf(ceilf(5.0f * sigma), 1.0f);
    int64_t radius = f32_to_isize(rf);
    float norm_scale = 1.0f;
    if (cfg->normalize_color) {
        float t = (float)size * cfg->pixel_size / (cfg->hi - cfg->lo);
        norm_scale = t * t;
    }
    const int64_t side = 2 * radius + 1;
    float* wbuf = (float*)malloc((size_t)(side * side) * sizeof(float));
    int64_t* xbuf = (int64_t*)malloc((size_t)(side * side) * sizeof(int64_t));
    if (!wbuf || !xbuf) return NPA_ERR_OUT_OF_MEMORY;
    for (uint64_t n = 0; n < count; ++n) {
        const float* pos = positions + 4 * n;
        const float* color = colors + 3 * n;
        float px = (pos[0] - cfg->lo) / (cfg->hi - cfg->lo) * ((float)size - 1.0f);
        float py = (pos[1] - cfg->lo) / (cfg->hi - cfg->lo) * ((float)size - 1.0f);
        if (cfg->y_up) py = ((float)size - 1.0f) - py;
        int64_t bx = f32_to_isize(floorf(px)), by = f32_to_isize(floorf(py));
        float fx = px - (float)bx, fy = py - (float)by;
        size_t nw = 0;
        float weight_sum = 0.0f;
        for (int64_t oy = -radius; oy <= radius; ++oy)
            for (int64_t ox = -radius; ox <= radius; ++ox) {
                int64_t x = bx + ox, y = by + oy;
                if (x < 0 || y < 0 || x >= size || y >= size) continue;
                float dx = (float)ox - fx, dy = (float)oy - fy;
                float w = expf(-(dx * dx + dy * dy) / (2.0f * sigma * sigma));
                wbuf[nw] = w;
                xbuf[nw] = y * size + x;
                ++nw;
                weight_sum += w;
            }
        float denom = cfg->normalize_color ? fmaxf(weight_sum, 1e-8f) : 1.0f;
        for (size_t k = 0; k < nw; ++k) {
            float w = wbuf[k] / denom * norm_scale;
            float* px4 = image + 4 * xbuf[k];
            px4[0] += color[0] * w;
            px4[1] += color[1] * w;
            px4[2] += color[2] * w;
            px4[3] += w;
        }
    }
    free(wbuf);
    free(xbuf);
    return NPA_OK;
}

/* ------------------------------------------------------------ 3D render raster
 * crates/burn_automata/src/render_loss/{math,projection,attributes,image}.rs */
#define RENDER_EPS 1.0e-8f

static float render_dot3(const float* p4, const float* r3) { /* math.rs:20-22 */
    return p4[0] * r3[0] + p4[1] * r3[1] + p4[2] * r3[2];
}

static void render_normalize3(const float v[3], float out[3]) { /* math.rs:32-39 */
    float norm = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    if (norm <= RENDER_EPS) {
        out[0] = 0.0f;
        out[1] = 0.0f;
        out[2] = 1.0f;
        return;
    }
    out[0] = v[0] / norm;
    out[1] = v[1] / norm;
    out[2] = v[2] / norm;
}

static float render_sigmoid(float v) { /* math.rs:11-18 */
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    float e = expf(v);
    return e / (1.0f + e);
}

/* view_basis (projection.rs:31-43); cross3 as math.rs:24-30. */
int oracle_view_basis(uint32_t view, float right[3], float up[3], float forward[3]) {
    static const float I[3][3] = {{1.0f, 0.0f, 0.0f}, {0.0f, 1.0f, 0.0f}, {0.0f, 0.0f, 1.0f}};
    const float* r;
    const float* u;
    const float* f;
    switch (view) {
        case NPA_VIEW_XY: r = I[0], u = I[1], f = I[2]; break;
        case NPA_VIEW_XZ: r = I[0], u = I[2], f = I[1]; break;
        case NPA_VIEW_YZ: r = I[1], u = I[2], f = I[0]; break;
        case NPA_VIEW_ISO: {
            const float a[3] = {1.0f, -1.0f, 0.0f}, b[3] = {1.0f, 1.0f, 2.0f};
            render_normalize3(a, right);
            render_normalize3(b, up);
            const float c[3] = {right[1] * up[2] - right[2] * up[1], right[2] * up[0] - right[0] * up[2],
                                right[0] * up[1] - right[1] * up[0]};
            render_normalize3(c, forward);
            return NPA_OK;
        }
        default: return NPA_ERR_INVALID_ARGUMENT;
    }
    memcpy(right, r, 12);
    memcpy(up, u, 12);
    memcpy(forward, f, 12);
    return NPA_OK;
}

/* project_positions (projection.rs:11-29): out[count][3] = (x, y, depth). */
int oracle_project_positions(uint32_t view, const float* positions, uint32_t count, float world_scale,
                             float* out) {
    float right[3], up[3], fwd[3];
    int st = oracle_view_basis(view, right, up, fwd);
    if (st) return st;
    for (uint64_t n = 0; n < count; ++n) {
        const float* p = positions + 4 * n;
        float depth = clamp_f32(0.5f + 0.5f * render_dot3(p, fwd) / fmaxf(world_scale, RENDER_EPS), 0.0f, 1.0f);
        out[3 * n] = render_dot3(p, right);
        out[3 * n + 1] = render_dot3(p, up);
        out[3 * n + 2] = depth;
    }
    return NPA_OK;
}

/* splat_projected (image.rs:18-79): image[size*size][5] = (r, g, b, alpha, depth_sum). */
int oracle_splat_projected(const float* projected, const float* colors, const float* opacities,
                           const float* sigmas, uint32_t count, const npa_render_cfg* cfg, float* image) {
    const int64_t size = cfg->image_size;
    memset(image, 0, (size_t)(size * size * 5) * sizeof(float));
    const float norm_scale = 1.0f / (float)(count > 1 ? count : 1);
    const float ws = cfg->world_scale;
    /* the largest footprint any particle can have: sigma <= max(max_sigma, EPS) */
    const int64_t rmax = f32_to_isize(fmaxf(ceilf(5.0f * fmaxf(cfg->max_sigma, RENDER_EPS)), 1.0f));
    const int64_t side = 2 * rmax + 1;
    float* wbuf = (float*)malloc((size_t)(side * side) * sizeof(float));
    int64_t* xbuf = (int64_t*)malloc((size_t)(side * side) * sizeof(int64_t));
    if (!wbuf || !xbuf) {
        free(wbuf);
        free(xbuf);
        return NPA_ERR_OUT_OF_MEMORY;
    }
    for (uint64_t n = 0; n < count; ++n) {
        const float* pp = projected + 3 * n;
        const float* color = colors + 3 * n;
        float sigma = fmaxf(clamp_f32(sigmas[n], cfg->min_sigma, cfg->max_sigma), RENDER_EPS);
        float sigma2 = sigma * sigma;
        int64_t radius = f32_to_isize(fmaxf(ceilf(5.0f * sigma), 1.0f));
        float px = (pp[0] + ws) / (2.0f * ws) * ((float)size - 1.0f);
        float py = (ws - pp[1]) / (2.0f * ws) * ((float)size - 1.0f);
        int64_t bx = f32_to_isize(floorf(px)), by = f32_to_isize(floorf(py));
        float fx = px - (float)bx, fy = py - (float)by;
        size_t nw = 0;
        float weight_sum = 0.0f;
        for (int64_t oy = -radius; oy <= radius; ++oy)
            for (int64_t ox = -radius; ox <= radius; ++ox) {
                int64_t x = bx + ox, y = by + oy;
                if (x < 0 || y < 0 || x >= size || y >= size) continue;
                float dx = (float)ox - fx, dy = (float)oy - fy;
                float w = expf(-(dx * dx + dy * dy) / (2.0f * sigma2));
                wbuf[nw] = w;
                xbuf[nw] = y * size + x;
                ++nw;
                weight_sum += w;
            }
        float denom = fmaxf(weight_sum, RENDER_EPS);
        float opacity = clamp_f32(opacities[n], 0.0f, 1.0f);
        for (size_t k = 0; k < nw; ++k) {
            float w = wbuf[k] / denom * norm_scale * opacity;
            float* px5 = image + 5 * xbuf[k];
            px5[0] += color[0] * w;
            px5[1] += color[1] * w;
            px5[2] += color[2] * w;
            px5[3] += w;
            px5[4] += pp[2] * w;
        }
    }
    free(wbuf);
    free(xbuf);
    return NPA_OK;
}

/* state_tail_render_attributes (attributes.rs:15-87) with growth_3d_material_opacity_channel
 * (crates/burn_automata/src/rollout/mod.rs:37-45: channel 8 when S > 8, else 3 when S > 3). */
int oracle_render_attributes(const float* states, uint32_t count, uint32_t state_dims, const npa_render_cfg* cfg,
                             float* colors, float* opacities, float* sigmas, float* derivatives) {
    if (state_dims < 3) return NPA_ERR_INVALID_ARGUMENT;
    if (cfg->gaussian_decode_mode == NPA_DECODE_SH0_LEARNED_SCALE && state_dims < 5) return NPA_ERR_INVALID_ARGUMENT;
    const uint32_t S = state_dims, tail = S - 3;
    const int opacity_ch = S > 8 ? 8 : (S > 3 ? 3 : -1);
    for (uint64_t i = 0; i < count; ++i) {
        const float* s = states + i * S;
        for (int k = 0; k < 3; ++k) colors[3 * i + k] = clamp_f32(s[tail + k] + 0.5f, 0.0f, 1.0f);
        opacities[i] = opacity_ch >= 0 ? clamp_f32(render_sigmoid(s[opacity_ch] + cfg->opacity_logit_bias), 0.001f, 0.95f)
                                       : 0.95f;
        float sigma, derivative = 0.0f;
        switch (cfg->gaussian_decode_mode) {
            case NPA_DECODE_PARTICLE_POINT: sigma = fmaxf(cfg->min_sigma, RENDER_EPS); break;
            case NPA_DECODE_SH0_LEARNED_SCALE: {
                float logit = clamp_f32(s[S - 5], -8.0f, 8.0f);
                float raw = cfg->sigma * expf(logit);
                sigma = clamp_f32(raw, cfg->min_sigma, cfg->max_sigma);
                derivative = (raw > cfg->min_sigma && raw < cfg->max_sigma) ? raw : 0.0f;
            } break;
            default: sigma = clamp_f32(cfg->sigma, cfg->min_sigma, cfg->max_sigma); break;
        }
        sigmas[i] = sigma;
        if (derivatives) derivatives[i] = derivative;
    }
    return NPA_OK;
}

/* ------------------------------------------------------------ perception adjoint
 * crates/burn_automata_kernels/src/reference/adjoint.rs, serial like the reference: every
 * accumulation into the adjoint arrays happens in the reference's order. */

/* smoothing_poly6_delta_adjoint  kernels.rs:62-79 */
static void poly6_delta_adjoint(const float delta[4], float r2, const npa_grid_cfg* cfg, float out_adj,
                                float out[4]) {
    out[0] = out[1] = out[2] = out[3] = 0.0f;
    float eps2 = cfg->eps * cfg->eps;
    if (r2 >= eps2) return;
    float x = eps2 - r2;
    float dk = -3.0f * poly6_norm(cfg) * x * x;
    for (uint32_t a = 0; a < cfg->dim; ++a) out[a] = out_adj * dk * 2.0f * delta[a];
}

/* spiky_gradient_delta_adjoint  kernels.rs:100-126 */
static void spiky_delta_adjoint(const float delta[4], float r2, const npa_grid_cfg* cfg, float coeff,
                                const float* out_adj, float out[4]) {
    out[0] = out[1] = out[2] = out[3] = 0.0f;
    float eps2 = cfg->eps * cfg->eps;
    if (r2 <= 0.0f || r2 >= eps2) return;
    float r = sqrtf(r2);
    float norm = coeff * spiky_norm(cfg) * 3.0f;
    float t = cfg->eps - r;
    float scale = norm * (t * t) / r;
    float dscale_dr = norm * (1.0f - (cfg->eps * cfg->eps) / r2);
    float dot = out_adj[0] * delta[0];
    for (uint32_t a = 1; a < cfg->dim; ++a) dot += out_adj[a] * delta[a];
    for (uint32_t a = 0; a < cfg->dim; ++a) out[a] = scale * out_adj[a] + dscale_dr * dot * delta[a] / r;
}

/* log_normalize_adjoint  normalize.rs:71-91 (adds into in_adj) */
static void log_normalize_adjoint(const float* in, const float* out_adj, float* in_adj, uint32_t n) {
    const float E = 1.0e-6f;
    float s = in[0] * in[0];
    for (uint32_t k = 1; k < n; ++k) s += in[k] * in[k];
    float norm = fmaxf(sqrtf(s + E * E), E);
    float scale = log1pf(norm) / norm;
    float dscale = (norm / (1.0f + norm) - log1pf(norm)) / (norm * norm);
    float dot = in[0] * out_adj[0];
    for (uint32_t k = 1; k < n; ++k) dot += in[k] * out_adj[k];
    float radial = dscale * dot / norm;
    for (uint32_t k = 0; k < n; ++k) in_adj[k] += scale * out_adj[k] + radial * in[k];
}

/* accumulate_volume_density_adjoint  adjoint.rs:420-431 */
static void volume_density_adjoint(const float* density, float* density_adj, uint64_t j, float v_adj) {
    float rho = density[j];
    if (fabsf(rho) <= 1.0e-20f || !isfinite(rho)) return;
    density_adj[j] -= v_adj / (rho * rho);
}

/* add_delta_position_adjoint  adjoint.rs:433-445 */
static void add_delta_position_adjoint(float* pos_adj, uint64_t lhs, uint64_t rhs, uint32_t dim,
                                       const float d_adj[4]) {
    for (uint32_t a = 0; a < dim; ++a) {
        pos_adj[4 * rhs + a] += d_adj[a];
        pos_adj[4 * lhs + a] -= d_adj[a];
    }
}

/* inverse_matrix_adjoint  adjoint.rs:447-468 (subtracts into m_adj) */
static void inverse_matrix_adjoint(const float inv[9], const float inv_adj[9], uint32_t d, float m_adj[9]) {
    for (uint32_t row = 0; row < d; ++row)
        for (uint32_t col = 0; col < d; ++col) {
            float v = 0.0f;
            for (uint32_t ir = 0; ir < d; ++ir)
                for (uint32_t ic = 0; ic < d; ++ic) v += inv[ir * d + row] * inv_adj[ir * d + ic] * inv[col * d + ic];
            m_adj[row * d + col] -= v;
        }
}

/* density_gradient_scale  adjoint.rs:470-489 */
static float density_gradient_scale(const npa_grid_cfg* cfg, const npa_perception_opts* o, uint32_t particle_count) {
    float eps0 = fmaxf(o->eps0, FLT_MIN);
    float s = o->scale_equivariance ? powi_f32(cfg->eps / eps0, 1 + (int)cfg->dim) : 1.0f;
    return s * (o->particle_density_equivariance ? 1.0f / (float)(particle_count > 1 ? particle_count : 1) : 1.0f);
}

/* perceive_adjoint_with_options  adjoint.rs:27-136 with accumulate_blurred_state_adjoint (138-166),
 * accumulate_state_gradient_adjoint (168-348), accumulate_density_gradient_position_adjoint
 * (350-397) and accumulate_density_kernel_position_adjoint (399-418). feature_adjoint
 * [total][F]; outputs state_adj [total][S], pos_adj [total][4] (overwritten). */
int oracle_perceive_adjoint(const float* positions, const float* states, uint32_t batch_size,
                            uint32_t particle_count, uint32_t S, const npa_grid_cfg* cfg,
                            const npa_perception_opts* o, const float* fadj, float* state_adj,
                            float* pos_adj) {
    int st = oracle_grid_validate(cfg);
    if (st) return st;
    const uint64_t total = (uint64_t)batch_size * particle_count;
    const uint32_t d = cfg->dim, F = oracle_feature_dims(S, d, o);
    hashgrid h;
    st = hashgrid_build(positions, batch_size, particle_count, cfg, &h);
    float* density = (float*)calloc(total + 1, sizeof(float));
    float* dens_adj = (float*)calloc(total + 1, sizeof(float));
    float* raw = (float*)calloc((size_t)S * d + 1, sizeof(float));
    float* rga = (float*)calloc((size_t)S * d + 1, sizeof(float));
    if (st || !density || !dens_adj || !raw || !rga) {
        hashgrid_free(&h);
        free(density);
        free(dens_adj);
        free(raw);
        free(rga);
        return st ? st : NPA_ERR_OUT_OF_MEMORY;
    }
    pass_density(positions, &h.view, cfg, NULL, total, density);
    memset(state_adj, 0, total * S * sizeof(float));
    memset(pos_adj, 0, total * 4 * sizeof(float));
    nbuf buf = {0};
    for (uint64_t idx = 0; idx < total; ++idx) {
        const float* fa = fadj + idx * F;
        uint32_t cur = 0;
        for (uint32_t c = 0; c < S; ++c) state_adj[idx * S + c] += fa[cur + c];
        cur += S;
        collect_neighbors(idx, positions, &h.view, cfg, &buf);
        /* blurred state (adjoint.rs:138-166) */
        const float* badj = fa + cur;
        for (size_t k = 0; k < buf.len; ++k) {
            const neighbor* n = &buf.v[k];
            float vol = recip_finite(density[n->j]);
            float kern = poly6(n->r2, cfg);
            float w = kern * vol;
            const float* sj = states + (uint64_t)n->j * S;
            float wadj = 0.0f;
            for (uint32_t c = 0; c < S; ++c) {
                state_adj[(uint64_t)n->j * S + c] += badj[c] * w;
                wadj += badj[c] * sj[c];
            }
            float da[4];
            poly6_delta_adjoint(n->delta, n->r2, cfg, wadj * vol, da);
            add_delta_position_adjoint(pos_adj, idx, n->j, d, da);
            volume_density_adjoint(density, dens_adj, n->j, wadj * kern);
        }
        cur += S;
        if (o->state_grad) { /* adjoint.rs:168-348 */
            const float* gadj = fa + cur;
            const float* si = states + idx * S;
            memset(raw, 0, (size_t)S * d * sizeof(float));
            float moment[9] = {0};
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (n->j == idx) continue;
                float vol = recip_finite(density[n->j]);
                float g[4];
                spiky_grad(n->delta, n->r2, cfg, vol, g);
                const float* sj = states + (uint64_t)n->j * S;
                for (uint32_t c = 0; c < S; ++c) {
                    float diff = sj[c] - si[c];
                    for (uint32_t a = 0; a < d; ++a) raw[c * d + a] += diff * g[a];
                }
                if (o->hybrid_state_gradient)
                    for (uint32_t r = 0; r < d; ++r)
                        for (uint32_t cc = 0; cc < d; ++cc) moment[r * d + cc] += n->delta[r] * g[cc];
            }
            float inv[9];
            if (o->hybrid_state_gradient) safe_inverse_symmetric(moment, d, inv);
            float scale = o->scale_equivariance ? cfg->eps / fmaxf(o->eps0, FLT_MIN) : 1.0f;
            float inv_adj[9] = {0};
            for (uint32_t c = 0; c < S; ++c) {
                float corr[4] = {0};
                const uint32_t gb = c * d;
                for (uint32_t a = 0; a < d; ++a) corr[a] = raw[gb + a];
                if (o->hybrid_state_gradient) {
                    float mc[4] = {0};
                    for (uint32_t oa = 0; oa < d; ++oa)
                        for (uint32_t ia = 0; ia < d; ++ia) mc[oa] += corr[ia] * inv[ia * d + oa];
                    memcpy(corr, mc, sizeof(corr));
                }
                float nin[4] = {0};
                for (uint32_t a = 0; a < d; ++a) nin[a] = corr[a] * scale;
                float cadj[4] = {0};
                if (o->log_norm_grad) log_normalize_adjoint(nin, gadj + gb, cadj, d);
                else
                    for (uint32_t a = 0; a < d; ++a) cadj[a] = gadj[gb + a];
                for (uint32_t a = 0; a < d; ++a) cadj[a] *= scale;
                float radj[4] = {0};
                if (o->hybrid_state_gradient) {
                    for (uint32_t ia = 0; ia < d; ++ia)
                        for (uint32_t oa = 0; oa < d; ++oa) radj[ia] += cadj[oa] * inv[ia * d + oa];
                } else {
                    for (uint32_t a = 0; a < d; ++a) radj[a] = cadj[a];
                }
                for (uint32_t a = 0; a < d; ++a) rga[gb + a] = radj[a];
                if (o->hybrid_state_gradient)
                    for (uint32_t ia = 0; ia < d; ++ia)
                        for (uint32_t oa = 0; oa < d; ++oa) inv_adj[ia * d + oa] += raw[gb + ia] * cadj[oa];
            }
            float madj[9] = {0};
            if (o->hybrid_state_gradient) inverse_matrix_adjoint(inv, inv_adj, d, madj);
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (n->j == idx) continue;
                float vol = recip_finite(density[n->j]);
                float vg[4], ug[4];
                spiky_grad(n->delta, n->r2, cfg, vol, vg);
                spiky_grad(n->delta, n->r2, cfg, 1.0f, ug);
                const float* sj = states + (uint64_t)n->j * S;
                for (uint32_t c = 0; c < S; ++c) {
                    const uint32_t gb = c * d;
                    float diff = sj[c] - si[c];
                    float sc = rga[gb] * vg[0];
                    for (uint32_t a = 1; a < d; ++a) sc += rga[gb + a] * vg[a];
                    state_adj[(uint64_t)n->j * S + c] += sc;
                    state_adj[idx * S + c] -= sc;
                    float gda[4] = {0};
                    for (uint32_t a = 0; a < d; ++a) gda[a] = rga[gb + a] * diff;
                    float da[4];
                    spiky_delta_adjoint(n->delta, n->r2, cfg, vol, gda, da);
                    add_delta_position_adjoint(pos_adj, idx, n->j, d, da);
                    float va = gda[0] * ug[0];
                    for (uint32_t a = 1; a < d; ++a) va += gda[a] * ug[a];
                    volume_density_adjoint(density, dens_adj, n->j, va);
                }
                if (o->hybrid_state_gradient) {
                    float dda[4] = {0}, gda[4] = {0};
                    for (uint32_t r = 0; r < d; ++r)
                        for (uint32_t cc = 0; cc < d; ++cc) {
                            float a = madj[r * d + cc];
                            dda[r] += a * vg[cc];
                            gda[cc] += a * n->delta[r];
                        }
                    float gd[4];
                    spiky_delta_adjoint(n->delta, n->r2, cfg, vol, gda, gd);
                    for (uint32_t a = 0; a < d; ++a) dda[a] += gd[a];
                    add_delta_position_adjoint(pos_adj, idx, n->j, d, dda);
                    float va = gda[0] * ug[0];
                    for (uint32_t a = 1; a < d; ++a) va += gda[a] * ug[a];
                    volume_density_adjoint(density, dens_adj, n->j, va);
                }
            }
            cur += S * d;
        }
        if (o->density_grad) { /* adjoint.rs:350-397 */
            const float* dadj = fa + cur;
            float rawd[4] = {0};
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (n->j == idx) continue;
                float g[4];
                spiky_grad(n->delta, n->r2, cfg, 1.0f, g);
                for (uint32_t a = 0; a < d; ++a) rawd[a] += g[a];
            }
            float scale = density_gradient_scale(cfg, o, particle_count);
            float nin[4] = {0};
            for (uint32_t a = 0; a < d; ++a) nin[a] = rawd[a] * scale;
            float radj[4] = {0};
            if (o->log_norm_density_grad) {
                log_normalize_adjoint(nin, dadj, radj, d);
                for (uint32_t a = 0; a < d; ++a) radj[a] *= scale;
            } else {
                for (uint32_t a = 0; a < d; ++a) radj[a] = dadj[a] * scale;
            }
            for (size_t k = 0; k < buf.len; ++k) {
                const neighbor* n = &buf.v[k];
                if (n->j == idx) continue;
                float da[4];
                spiky_delta_adjoint(n->delta, n->r2, cfg, 1.0f, radj, da);
                add_delta_position_adjoint(pos_adj, idx, n->j, d, da);
            }
            cur += d;
        }
        if (o->position_features)
            for (uint32_t a = 0; a < d; ++a) pos_adj[4 * idx + a] += fa[cur + a];
    }
    /* accumulate_density_kernel_position_adjoint (adjoint.rs:399-418) */
    for (uint64_t idx = 0; idx < total; ++idx) {
        float adj = dens_adj[idx];
        if (adj == 0.0f) continue;
        collect_neighbors(idx, positions, &h.view, cfg, &buf);
        for (size_t k = 0; k < buf.len; ++k) {
            const neighbor* n = &buf.v[k];
            float da[4];
            poly6_delta_adjoint(n->delta, n->r2, cfg, adj, da);
            add_delta_position_adjoint(pos_adj, idx, n->j, d, da);
        }
    }
    free(buf.v);
    hashgrid_free(&h);
    free(density);
    free(dens_adj);
    free(raw);
    free(rga);
    return NPA_OK;
}

/* ------------------------------------------------------------------ oriented Gaussian raster
 * The EWA raster of the planar Gaussian export, restated from the published 3D Gaussian
 * splatting forward pass (Kerbl et al. 2023, with the EWA splat projection of Zwicker et al.
 * 2001). The reference draws the export through bevy_gaussian_splatting 8.0.1 (Cargo.toml:23;
 * crates/bevy_automata/src/viewer/cloud.rs:80-97), which is not vendored: no reference test pins
 * these pixels (parity unpinned against the reference; pinned by closed forms in the tests).
 * Straightforward loops: each tile filters the depth-sorted Gaussians whose tile rectangle holds
 * it, and each of its pixels walks that list serially. */
typedef struct raster_splat {
    int live;
    float depth;
    float mx, my, qa, qb, qc, opacity, rgb[3];
    int tx0, tx1, ty0, ty1;
} raster_splat;

/* Real spherical harmonics in the sign convention of the 3DGS code (Condon-Shortley phase),
 * bands 0..3: 1/(2 sqrt(pi)), sqrt(3/(4 pi)), ... */
static const float kShC0 = 0.28209479177387814f;
static const float kShC1 = 0.4886025119029199f;
static const float kShC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                               -1.0925484305920792f, 0.5462742152960396f};
static const float kShC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                               0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                               -0.5900435899266435f};

static void raster_sh_color(const float* sh, uint32_t degree, const float dir[3], float out[3]) {
    const float x = dir[0], y = dir[1], z = dir[2];
    float basis[16];
    basis[0] = kShC0;
    if (degree > 0) {
        basis[1] = -kShC1 * y;
        basis[2] = kShC1 * z;
        basis[3] = -kShC1 * x;
    }
    if (degree > 1) {
        const float xx = x * x, yy = y * y, zz = z * z;
        basis[4] = kShC2[0] * (x * y);
        basis[5] = kShC2[1] * (y * z);
        basis[6] = kShC2[2] * (2.0f * zz - xx - yy);
        basis[7] = kShC2[3] * (x * z);
        basis[8] = kShC2[4] * (xx - yy);
        if (degree > 2) {
            basis[9] = kShC3[0] * y * (3.0f * xx - yy);
            basis[10] = kShC3[1] * (x * y) * z;
            basis[11] = kShC3[2] * y * (4.0f * zz - xx - yy);
            basis[12] = kShC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
            basis[13] = kShC3[4] * x * (4.0f * zz - xx - yy);
            basis[14] = kShC3[5] * z * (xx - yy);
            basis[15] = kShC3[6] * x * (xx - 3.0f * yy);
        }
    }
    const uint32_t K = (degree + 1) * (degree + 1);
    for (int ch = 0; ch < 3; ++ch) {
        float acc = 0.0f;
        for (uint32_t k = 0; k < K; ++k) acc += basis[k] * sh[k * 3 + ch];
        acc += 0.5f;
        out[ch] = acc > 0.0f ? acc : 0.0f;
    }
}

static float raster_clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void raster_prepare(const float* pv, const float* sh, const float* rot, const float* so,
                           const npa_raster_camera* cam, const float campos[3], uint32_t tiles_x,
                           uint32_t tiles_y, raster_splat* out) {
    const float* V = cam->view;
    out->live = 0;
    if (!(pv[3] > 0.0f)) return;
    const float vx = V[0] * pv[0] + V[1] * pv[1] + V[2] * pv[2] + V[3];
    const float vy = V[4] * pv[0] + V[5] * pv[1] + V[6] * pv[2] + V[7];
    const float vz = V[8] * pv[0] + V[9] * pv[1] + V[10] * pv[2] + V[11];
    /* the 3DGS camera frame: x right, y down, z forward */
    const float tx = vx, ty = -vy, tz = -vz;
    if (!(tz > cam->near_plane) || !(tz <= cam->far_plane)) return;
    float qw = rot[0], qx = rot[1], qy = rot[2], qz = rot[3];
    const float qn = sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
    if (qn > 0.0f && qn < INFINITY) {
        qw /= qn; qx /= qn; qy /= qn; qz /= qn;
    } else {
        qw = 1.0f; qx = qy = qz = 0.0f;
    }
    const float R[3][3] = {
        {1.0f - 2.0f * (qy * qy + qz * qz), 2.0f * (qx * qy - qw * qz), 2.0f * (qx * qz + qw * qy)},
        {2.0f * (qx * qy + qw * qz), 1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz - qw * qx)},
        {2.0f * (qx * qz - qw * qy), 2.0f * (qy * qz + qw * qx), 1.0f - 2.0f * (qx * qx + qy * qy)}};
    float M[3][3];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) M[r][c] = R[r][c] * so[c];
    float S[3][3];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) S[r][c] = M[r][0] * M[c][0] + M[r][1] * M[c][1] + M[r][2] * M[c][2];
    /* view rotation in the 3DGS frame */
    const float W[3][3] = {{V[0], V[1], V[2]}, {-V[4], -V[5], -V[6]}, {-V[8], -V[9], -V[10]}};
    const float limx = 1.3f * fmaxf(cam->cx, (float)cam->width - cam->cx) / cam->fx;
    const float limy = 1.3f * fmaxf(cam->cy, (float)cam->height - cam->cy) / cam->fy;
    const float jx = raster_clampf(tx / tz, -limx, limx) * tz;
    const float jy = raster_clampf(ty / tz, -limy, limy) * tz;
    const float J[2][3] = {{cam->fx / tz, 0.0f, -(cam->fx * jx) / (tz * tz)},
                           {0.0f, cam->fy / tz, -(cam->fy * jy) / (tz * tz)}};
    float T[2][3];
    for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 3; ++c) T[r][c] = J[r][0] * W[0][c] + J[r][1] * W[1][c] + J[r][2] * W[2][c];
    float U[2][3];
    for (int r = 0; r < 2; ++r)
        for (int c = 0; c < 3; ++c) U[r][c] = T[r][0] * S[0][c] + T[r][1] * S[1][c] + T[r][2] * S[2][c];
    const float a = (U[0][0] * T[0][0] + U[0][1] * T[0][1] + U[0][2] * T[0][2]) + 0.3f;
    const float b = U[0][0] * T[1][0] + U[0][1] * T[1][1] + U[0][2] * T[1][2];
    const float c = (U[1][0] * T[1][0] + U[1][1] * T[1][1] + U[1][2] * T[1][2]) + 0.3f;
    const float det = a * c - b * b;
    if (!(det > 0.0f) || !(det < INFINITY)) return;
    const float mid = 0.5f * (a + c);
    const float lam = mid + sqrtf(fmaxf(0.1f, mid * mid - det));
    const float radius = ceilf(3.0f * sqrtf(lam));
    const float mx = cam->cx + cam->fx * tx / tz;
    const float my = cam->cy + cam->fy * ty / tz;
    if (!(fabsf(mx) < 1e30f) || !(fabsf(my) < 1e30f) || !(radius < 1e30f)) return;
    const float fx0 = raster_clampf(floorf((mx - radius) / 16.0f), 0.0f, (float)tiles_x);
    const float fx1 = raster_clampf(floorf((mx + radius) / 16.0f) + 1.0f, 0.0f, (float)tiles_x);
    const float fy0 = raster_clampf(floorf((my - radius) / 16.0f), 0.0f, (float)tiles_y);
    const float fy1 = raster_clampf(floorf((my + radius) / 16.0f) + 1.0f, 0.0f, (float)tiles_y);
    out->tx0 = (int)fx0; out->tx1 = (int)fx1; out->ty0 = (int)fy0; out->ty1 = (int)fy1;
    if (out->tx0 >= out->tx1 || out->ty0 >= out->ty1) return;
    /* the conic scaled so that power * log2(e) = qa dx^2 + qc dy^2 + qb dx dy */
    const float L = 1.4426950408889634f;
    out->qa = (c / det) * (-0.5f * L);
    out->qb = (-b / det) * -L;
    out->qc = (a / det) * (-0.5f * L);
    out->mx = mx;
    out->my = my;
    out->depth = tz;
    out->opacity = so[3];
    if (cam->color_mode == NPA_RASTER_COLOR_RGB) {
        for (int ch = 0; ch < 3; ++ch) out->rgb[ch] = sh[ch];
    } else {
        float d[3] = {pv[0] - campos[0], pv[1] - campos[1], pv[2] - campos[2]};
        const float dn = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
        for (int k = 0; k < 3; ++k) d[k] = dn > 0.0f ? d[k] / dn : 0.0f;
        raster_sh_color(sh, cam->sh_degree, d, out->rgb);
    }
    out->live = 1;
}

static const raster_splat* g_raster_sort_base;
static int raster_depth_order(const void* pa, const void* pb) {
    const uint32_t ia = *(const uint32_t*)pa, ib = *(const uint32_t*)pb;
    const float da = g_raster_sort_base[ia].depth, db = g_raster_sort_base[ib].depth;
    if (da < db) return -1;
    if (da > db) return 1;
    return ia < ib ? -1 : (ia > ib ? 1 : 0);
}

int oracle_raster_camera_center(const npa_raster_camera* cam, float out[3]) {
    /* view = [R | t] -> centre = -R^T t */
    const float* V = cam->view;
    for (int k = 0; k < 3; ++k) out[k] = -(V[k] * V[3] + V[4 + k] * V[7] + V[8 + k] * V[11]);
    return 0;
}

int oracle_raster_gaussians_3d(const float* position_visibility, const float* spherical_harmonic,
                               const float* rotation, const float* scale_opacity, uint32_t count,
                               const npa_raster_camera* cam, float* image, uint64_t* evaluated) {
    if (!cam || cam->width == 0 || cam->height == 0 || cam->sh_degree > 3 ||
        cam->color_mode > NPA_RASTER_COLOR_RGB || !(cam->near_plane > 0.0f) ||
        !(cam->far_plane > cam->near_plane))
        return NPA_ERR_INVALID_ARGUMENT;
    const uint32_t K = (cam->sh_degree + 1) * (cam->sh_degree + 1);
    const uint32_t tiles_x = (cam->width + 15) / 16, tiles_y = (cam->height + 15) / 16;
    float campos[3];
    oracle_raster_camera_center(cam, campos);
    raster_splat* sp = (raster_splat*)calloc(count ? count : 1, sizeof(raster_splat));
    uint32_t* order = (uint32_t*)malloc((count ? count : 1) * sizeof(uint32_t));
    if (!sp || !order) {
        free(sp);
        free(order);
        return NPA_ERR_OUT_OF_MEMORY;
    }
    uint32_t live = 0;
    for (uint32_t i = 0; i < count; ++i) {
        raster_prepare(position_visibility + 4ull * i, spherical_harmonic + (uint64_t)i * K * 3,
                       rotation + 4ull * i, scale_opacity + 4ull * i, cam, campos, tiles_x, tiles_y, &sp[i]);
        if (sp[i].live) order[live++] = i;
    }
    g_raster_sort_base = sp;
    qsort(order, live, sizeof(uint32_t), raster_depth_order);
    int oom = 0;
    uint64_t pairs = 0;
#pragma omp parallel reduction(+ : pairs)
    {
        uint32_t* list = (uint32_t*)malloc((live ? live : 1) * sizeof(uint32_t));
        if (!list) {
#pragma omp atomic write
            oom = 1;
        }
#pragma omp for schedule(dynamic, 1)
        for (uint32_t t = 0; t < tiles_x * tiles_y; ++t) {
            if (!list) continue;
            const int tx = (int)(t % tiles_x), ty = (int)(t / tiles_x);
            /* the tile's Gaussians, front to back */
            uint32_t n = 0;
            for (uint32_t k = 0; k < live; ++k) {
                const raster_splat* g = &sp[order[k]];
                if (tx >= g->tx0 && tx < g->tx1 && ty >= g->ty0 && ty < g->ty1) list[n++] = order[k];
            }
            for (uint32_t py = (uint32_t)ty * 16; py < (uint32_t)ty * 16 + 16 && py < cam->height; ++py)
                for (uint32_t px = (uint32_t)tx * 16; px < (uint32_t)tx * 16 + 16 && px < cam->width; ++px) {
                    float T = 1.0f, rgb[3] = {0.0f, 0.0f, 0.0f};
                    const float pxc = (float)px + 0.5f, pyc = (float)py + 0.5f;
                    for (uint32_t k = 0; k < n; ++k) {
                        const raster_splat* g = &sp[list[k]];
                        ++pairs;
                        const float dx = g->mx - pxc, dy = g->my - pyc;
                        const float p2 = fmaf(g->qa * dx, dx, fmaf(g->qc * dy, dy, g->qb * dx * dy));
                        if (p2 > 0.0f) continue;
                        const float alpha = fminf(0.99f, g->opacity * exp2f(p2));
                        if (alpha < 1.0f / 255.0f) continue;
                        const float next = T * (1.0f - alpha);
                        if (next < 0.0001f) break;
                        const float wgt = alpha * T;
                        for (int ch = 0; ch < 3; ++ch) rgb[ch] = fmaf(g->rgb[ch], wgt, rgb[ch]);
                        T = next;
                    }
                    float* o = image + 4 * ((uint64_t)py * cam->width + px);
                    o[0] = rgb[0];
                    o[1] = rgb[1];
                    o[2] = rgb[2];
                    o[3] = 1.0f - T;
                }
        }
        free(list);
    }
    if (evaluated) *evaluated = pairs;
    if (oom) {
        free(sp);
        free(order);
        return NPA_ERR_OUT_OF_MEMORY;
    }
    free(sp);
    free(order);
    return NPA_OK;
}
