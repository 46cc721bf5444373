/* A C caller of libnpa_hip.so through include/npa_abi.h alone (no Python): one fused step in
 * host-I/O mode (npa_step, the twin of NpaModel::step_cpu) and a resident rollout
 * (npa_state_create / npa_state_step / npa_state_read), on inputs read from raw float32 files.
 *
 * usage: c_step DIR N S H STEPS
 *   DIR/positions.f32 [N][4], DIR/states.f32 [N][S], DIR/w1.f32 [H][F], DIR/b1.f32 [H],
 *   DIR/w2.f32 [O][H], DIR/b2.f32 [O], DIR/mask.f32 [N]  (F = 4S, O = 2 + S: the C1 model)
 * writes DIR/step_positions.f32, DIR/step_states.f32, DIR/step_density.f32 (the masked step) and
 * DIR/roll_positions.f32, DIR/roll_states.f32 (STEPS resident steps, device hash mask p = 0.5,
 * seed 42). Exit status 0 on success; a failing call prints its status and message. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/npa_abi.h"

static float* read_f32(const char* dir, const char* name, size_t count) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(2);
    }
    float* v = (float*)malloc(count * sizeof(float));
    if (!v || fread(v, sizeof(float), count, f) != count) {
        fprintf(stderr, "short read %s\n", path);
        exit(2);
    }
    fclose(f);
    return v;
}

static void write_f32(const char* dir, const char* name, const float* v, size_t count) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE* f = fopen(path, "wb");
    if (!f || fwrite(v, sizeof(float), count, f) != count) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(2);
    }
    fclose(f);
}

#define CHECK(ctx, call)                                                                   \
    do {                                                                                   \
        npa_status st_ = (call);                                                           \
        if (st_ != NPA_OK) {                                                               \
            fprintf(stderr, "%s -> %d: %s\n", #call, (int)st_, npa_last_error(ctx));       \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

int main(int argc, char** argv) {
    if (argc != 6) {
        fprintf(stderr, "usage: %s DIR N S H STEPS\n", argv[0]);
        return 2;
    }
    const char* dir = argv[1];
    const uint32_t n = (uint32_t)strtoul(argv[2], NULL, 10), s = (uint32_t)strtoul(argv[3], NULL, 10);
    const uint32_t h = (uint32_t)strtoul(argv[4], NULL, 10), steps = (uint32_t)strtoul(argv[5], NULL, 10);
    const uint32_t f = 4 * s, o = 2 + s;

    float* pos = read_f32(dir, "positions.f32", (size_t)n * 4);
    float* st = read_f32(dir, "states.f32", (size_t)n * s);
    float* w1 = read_f32(dir, "w1.f32", (size_t)h * f);
    float* b1 = read_f32(dir, "b1.f32", h);
    float* w2 = read_f32(dir, "w2.f32", (size_t)o * h);
    float* b2 = read_f32(dir, "b2.f32", o);
    float* mask = read_f32(dir, "mask.f32", n);

    /* the C1 configuration: HashGridConfig Particle 64x64, eps 0.05, clamped; growing-2D model with
     * eps0 0.05, density gradient off, state gradient on, ParticleDensityAndScale */
    npa_grid_cfg grid = {2, NPA_BOUNDARY_CLAMPED, NPA_MODE_PARTICLE, {64, 64, 1}, 0.05f, 32};
    npa_model_cfg model = {2, s, h, 0.05f, 0.5f, 0, 1, 1, 1, NPA_EQUIV_PARTICLE_DENSITY_AND_SCALE, 0};
    npa_weights weights = {w1, b1, w2, b2};

    npa_context* ctx = NULL;
    if (npa_context_create(0, NULL, &ctx) != NPA_OK) {
        fprintf(stderr, "npa_context_create failed\n");
        return 1;
    }
    CHECK(ctx, npa_context_set_host_io(ctx, 1));

    float* out_pos = (float*)malloc((size_t)n * 4 * sizeof(float));
    float* out_st = (float*)malloc((size_t)n * s * sizeof(float));
    float* dens = (float*)malloc((size_t)n * sizeof(float));
    CHECK(ctx, npa_step(ctx, pos, st, 1, n, &grid, &model, &weights, 1.0f, mask, out_pos, out_st, dens));
    write_f32(dir, "step_positions.f32", out_pos, (size_t)n * 4);
    write_f32(dir, "step_states.f32", out_st, (size_t)n * s);
    write_f32(dir, "step_density.f32", dens, n);

    npa_state* state = NULL;
    CHECK(ctx, npa_state_create(ctx, &model, &weights, &grid, pos, st, 1, n, 1.0f, 0.5f, 42, &state));
    CHECK(ctx, npa_state_step(state, steps));
    uint64_t k = 0;
    CHECK(ctx, npa_state_step_index(state, &k));
    if (k != steps) {
        fprintf(stderr, "step index %llu != %u\n", (unsigned long long)k, steps);
        return 1;
    }
    CHECK(ctx, npa_state_read(state, out_pos, out_st, NULL));
    write_f32(dir, "roll_positions.f32", out_pos, (size_t)n * 4);
    write_f32(dir, "roll_states.f32", out_st, (size_t)n * s);
    npa_state_destroy(state);
    npa_context_destroy(ctx);
    printf("c_step: %s, %u particles, one step and %u resident steps\n", npa_version(), n, steps);
    free(pos); free(st); free(w1); free(b1); free(w2); free(b2); free(mask);
    free(out_pos); free(out_st); free(dens);
    return 0;
}
