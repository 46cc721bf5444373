// npa_neighbors.hpp - neighbour-cell lookups shared by the neighbour passes (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "npa_internal.hpp"

namespace npa {

// A neighbour cell's run is walked in chunks of kNbChunk consecutive slots; the density pass
// records one accept mask per chunk.
constexpr int kNbChunk = 64;

__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// Candidate slots of neighbour cell (n0, n1, n2) of system b: in Particle mode the cell's own run
// of its split bin (no coordinate test needed) or, for an unsplit bin, the whole bin with
// `filter` set; in Grid mode the cell's bin. False when the cell holds no particle.
__device__ __forceinline__ bool cell_range(const StepParams& P, const uint32_t* __restrict__ bo, uint32_t b,
                                           int64_t n0, int64_t n1, int64_t n2, uint32_t& beg, uint32_t& end,
                                           bool& filter) {
    uint32_t cell;
    if (!cell_index(n0, n1, n2, P.g, &cell)) return false;
    const uint64_t bin = (uint64_t)b * P.g.cells + cell;
    filter = false;
    if (P.g.mode != 1) {
        beg = bo[bin];
        end = bo[bin + 1];
        return beg < end;
    }
    // the bin's directory size, its first entry and its end: all that a bin of one cell (most
    // bins) needs
    const int4* e = P.dir_e + bin * kDirGroups;
    const uint32_t nd = P.dir_n[bin];
    const int4 e0 = e[0];
    const uint32_t last = bo[bin + 1];
    if (nd == 0) return false;
    if (nd > kDirGroups) {
        beg = bo[bin];
        end = last;
        filter = true;
        return true;
    }
    if (nd == 1) {
        if ((int64_t)e0.x != n0 || (int64_t)e0.y != n1 || (int64_t)e0.z != n2) return false;
        beg = (uint32_t)e0.w;
        end = last;
        return true;
    }
    // several cells: the directory entries are loaded four at a time (each half's loads issued
    // together); a run ends where the next entry's run starts, the last one at the bin's end
    bool found = false;
    int hit_k = -1;
#pragma unroll
    for (uint32_t h = 0; h < kDirGroups; h += 4) {
        if (h >= nd) break;
        int4 ek[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) ek[k] = h + k < nd ? e[h + k] : make_int4(0, 0, 0, 0);
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            const bool hit = !found && h + k < nd && (int64_t)ek[k].x == n0 && (int64_t)ek[k].y == n1 &&
                             (int64_t)ek[k].z == n2;
            if (hit) {
                beg = (uint32_t)ek[k].w;
                hit_k = (int)(h + k);
                found = true;
            }
        }
    }
    if (found) end = (uint32_t)hit_k + 1 < nd ? (uint32_t)e[hit_k + 1].w : last;
    return found;
}

// cell_range for NU cells of one lane at once: every cell's directory loads (its size, first
// entry and end; a Grid-mode cell's start and end) are issued before the first is used, so the
// lookups cost one memory round trip instead of NU. A cell not wanted, outside a clamped grid or
// empty gets beg = end = 0. Bins of several cells (rare) finish through cell_range.
template <int NU>
__device__ __forceinline__ void cell_ranges(const StepParams& P, const uint32_t* __restrict__ bo, uint32_t b,
                                            const int64_t (&n)[NU][3], const bool (&want)[NU], uint32_t (&beg)[NU],
                                            uint32_t (&end)[NU], bool (&filter)[NU]) {
    uint64_t bin[NU];
    bool ok[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        uint32_t cell = 0;
        ok[u] = want[u] && cell_index(n[u][0], n[u][1], n[u][2], P.g, &cell);
        bin[u] = (uint64_t)b * P.g.cells + cell;
        beg[u] = 0;
        end[u] = 0;
        filter[u] = false;
    }
    if (P.g.mode != 1) {
        uint32_t lo[NU], hi[NU];
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            lo[u] = ok[u] ? bo[bin[u]] : 0u;
            hi[u] = ok[u] ? bo[bin[u] + 1] : 0u;
        }
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            beg[u] = lo[u];
            end[u] = hi[u];
        }
        return;
    }
    uint32_t nd[NU], last[NU];
    int4 e0[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        nd[u] = ok[u] ? P.dir_n[bin[u]] : 0u;
        e0[u] = ok[u] ? P.dir_e[bin[u] * kDirGroups] : make_int4(0, 0, 0, 0);
        last[u] = ok[u] ? bo[bin[u] + 1] : 0u;
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        if (nd[u] == 1) {
            if ((int64_t)e0[u].x == n[u][0] && (int64_t)e0[u].y == n[u][1] && (int64_t)e0[u].z == n[u][2]) {
                beg[u] = (uint32_t)e0[u].w;
                end[u] = last[u];
            }
        } else if (nd[u] != 0) {
            uint32_t bb = 0, ee = 0;
            bool ff = false;
            if (cell_range(P, bo, b, n[u][0], n[u][1], n[u][2], bb, ee, ff)) {
                beg[u] = bb;
                end[u] = ee;
                filter[u] = ff;
            }
        }
    }
}

// The candidate runs of the 3^D neighbour cells of cell (c0, c1, c2) of system b, looked up in
// parallel: lane k < 3^D takes neighbour k in the reference's visit order (k = (dz+1)*9 +
// (dy+1)*3 + (dx+1): dz, then dy, then dx). found: the cell holds particles.
template <int D>
__device__ __forceinline__ void neighbor_runs(const StepParams& P, const uint32_t* __restrict__ bo, uint32_t b,
                                              int c0, int c1, int c2, uint32_t lane, uint32_t& beg, uint32_t& end,
                                              bool& filter, bool& found) {
    constexpr uint32_t NC = D == 3 ? 27 : 9;
    beg = end = 0;
    filter = false;
    found = false;
    if (lane >= NC) return;
    const int dx = (int)(lane % 3) - 1, dy = (int)((lane / 3) % 3) - 1, dz = D == 3 ? (int)(lane / 9) - 1 : 0;
    found = cell_range(P, bo, b, (int64_t)c0 + dx, (int64_t)c1 + dy, (int64_t)c2 + dz, beg, end, filter);
}

}  // namespace npa
