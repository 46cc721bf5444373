// npa_hashgrid.hip - stable counting-sort hashgrid build on gfx950.
//
// Replaces build_hashgrid (crates/burn_automata_kernels/src/hashgrid.rs:16-69), bit-exact:
// bin_offsets = exclusive prefix of per-bin counts, and inside each bin the particles
// keep ascending original index (the reference's serial stable scatter).
//
// Kernels per build:
//   k_hash_rank    one block = one tile of `waves*R*64` consecutive particles of one
//                  system. Each wave walks its contiguous slice in rounds of 64: the cell
//                  key of each lane, its peers (lanes with the same key) from
//                  ceil(log2 C) wavefront ballots, the rank among peers by popcount, and
//                  a per-wave LDS counter per key (u16) carried across rounds. After a
//                  barrier, ranks are offset by the earlier waves' counters and the tile's
//                  per-key histogram row is written to table[tile][key].
//   k_table_offsets_scan  per key, exclusive prefix over the system's tiles (column scan);
//                  per block of 256 keys, the prefix of the earlier blocks' key totals from
//                  their published sums (one pass) -> bin_offsets. The generic key sorts
//                  run the two scans as k_table_scan and k_offsets_scan.
//   k_scatter      dst = bin_offsets[key] + table[tile][key] + rank; writes the
//                  permutation and its inverse. The rollout step's k_scatter_payload also
//                  writes the sorted particle records and state rows the neighbour passes
//                  read, and k_split then orders the bins that hold several cells by cell.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "npa_internal.hpp"

namespace npa {

// ------------------------------------------------------------------ DevBuf
hipError_t DevBuf::reserve(size_t want) {
    if (want <= bytes && ptr) return hipSuccess;
    release();
    size_t b = want ? want : 16;
    hipError_t e = hipMalloc(&ptr, b);
    if (e != hipSuccess) {
        ptr = nullptr;
        bytes = 0;
        return e;
    }
    bytes = b;
    return hipSuccess;
}

void DevBuf::release() {
    if (ptr && owned) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
    owned = true;
}

void DevBuf::view(void* p, size_t b) {
    release();
    ptr = p;
    bytes = b;
    owned = false;
}

// Every buffer of a hashgrid + step pass with its size, in one list for both set-ups (allocation
// and carving); the coordinate-overflow flags are handled by each set-up itself.
template <class F>
static void each_buffer(Workspace& w, const HashgridPlan& plan, uint64_t total, uint32_t batch, uint32_t state_dims,
                        int dim, uint32_t feature_dims, uint64_t wpad_bytes, F&& f) {
    const uint64_t t1 = total ? total : 1;
    const uint64_t bins = (uint64_t)batch * plan.cells;
    f(w.keys, t1 * 4);
    f(w.ranks, t1 * 4);
    f(w.table, (plan.table_entries ? plan.table_entries : 1) * 4);
    f(w.totals, (bins ? bins : 1) * 4);
    f(w.bin_offsets, (bins + 1) * 4);
    f(w.perm, t1 * 4);
    f(w.inv, t1 * 4);
    f(w.wl_count, 4 * kWlWords);
    f(w.worklist, (plan.worklist_cap + 1) * 8);
    // second-pass items: at most one partial item per (64-slot window, cell run) pair
    f(w.act_rows, t1 * 4);
    // sorted records: 64 slots of padding past the last particle, so a pass may load a whole
    // 64-slot chunk from any run start without clamping the index
    f(w.srec, (t1 + 64) * 16);
    f(w.scoord, dim == 3 ? (t1 + 64) * 16 : 16);
    f(w.sstate, t1 * (uint64_t)state_stride_for(state_dims ? state_dims : 1) * 4);
    f(w.svol, t1 * 16);
    f(w.counters, 64);
    f(w.features, t1 * (uint64_t)(feature_dims ? feature_dims : 1) * 4);
    f(w.wpad, wpad_bytes ? wpad_bytes : 4);
    f(w.tmpidx, t1 * 4);
    // two status words per 256-key block (the folded scan's second one) and the blocks' ticket
    f(w.scan_status, (uint64_t)batch * ((plan.cells + 255) / 256) * 16 + 8);
    f(w.tile_span, (uint64_t)batch * plan.tiles_per_sys * 32);
    f(w.dir_n, (bins ? bins : 1) * 4);
    f(w.bin_list, (bins ? bins : 1) * 4);
    f(w.dir_e, (bins ? bins : 1) * kDirGroups * 16);
    f(w.row_of, t1 * 4);
    f(w.nb_base, t1 * max_chunks(dim) * 4);
    f(w.nb_mask, t1 * max_chunks(dim) * 8);
    f(w.nb_count, t1 * 4);
    f(w.bin_count, (uint64_t)(plan.cells ? plan.cells : 1) * 8 + 32);
    f(w.bin_urow, t1 * 4);
}

hipError_t Workspace::reserve(const HashgridPlan& plan, uint64_t total, uint32_t batch,
                              uint32_t state_dims, int dim, uint32_t feature_dims) {
    hipError_t e = hipSuccess;
    const void* counters_before = bin_count.ptr;
    const size_t counter_bytes_before = bin_count.bytes;
    each_buffer(*this, plan, total, batch, state_dims, dim, feature_dims, 4, [&](DevBuf& b, uint64_t n) {
        if (e == hipSuccess) e = b.reserve((size_t)n);
    });
    if (e != hipSuccess) return e;
    // a new counter buffer starts at zero (complete before any stream uses it)
    if (bin_count.ptr != counters_before || bin_count.bytes != counter_bytes_before) {
        if ((e = hipMemset(bin_count.ptr, 0, bin_count.bytes)) != hipSuccess) return e;
        if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    }
    if (!flags.ptr) {
        if ((e = flags.reserve(64)) != hipSuccess) return e;
        if ((e = hipMemset(flags.ptr, 0, 64)) != hipSuccess) return e;
    }
    return hipSuccess;
}

uint64_t Workspace::carve(const HashgridPlan& plan, uint64_t total, uint32_t batch, uint32_t state_dims, int dim,
                          uint32_t feature_dims, uint64_t wpad_bytes, void* base, uint64_t capacity) {
    constexpr uint64_t kAlign = 256;
    uint64_t off = kCarveFlagBytes;  // the flags take the first 256 bytes
    each_buffer(*this, plan, total, batch, state_dims, dim, feature_dims, wpad_bytes, [&](DevBuf&, uint64_t n) {
        off += (n + kAlign - 1) / kAlign * kAlign;
    });
    if (off > capacity || !base) return off;
    char* p = static_cast<char*>(base);
    flags.view(p, kCarveFlagBytes);
    off = kCarveFlagBytes;
    each_buffer(*this, plan, total, batch, state_dims, dim, feature_dims, wpad_bytes, [&](DevBuf& b, uint64_t n) {
        b.view(p + off, (size_t)n);
        off += (n + kAlign - 1) / kAlign * kAlign;
    });
    return off;
}

void Workspace::release() {
    for (DevBuf* b : {&keys, &ranks, &table, &totals, &bin_offsets, &perm, &inv, &flags, &wl_count,
                      &worklist, &srec, &scoord, &sstate, &svol, &counters, &features, &wpad, &tmpidx,
                      &dir_n, &dir_e, &bin_list, &act_rows, &row_of, &nb_base, &nb_mask, &nb_count, &scan_status,
                      &tile_span, &bin_count, &bin_urow})
        b->release();
}

// ------------------------------------------------------------------- plan
float host_powi(float x, int n) {  // f32::powi, see oracle powi_f32 for the derivation
    bool recip = n < 0;
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

GridParams make_grid_params(const npa_grid_cfg& cfg) {
    GridParams g{};
    g.dim = (int)cfg.dim;
    g.boundary = (int)cfg.boundary;
    g.mode = (int)cfg.mode;
    uint32_t cells = 1;
    for (int a = 0; a < 3; ++a) g.size[a] = cfg.grid_size[a];
    for (uint32_t a = 0; a < cfg.dim; ++a) cells *= cfg.grid_size[a];
    g.cells = cells;
    g.eps = cfg.eps;
    g.eps2 = cfg.eps * cfg.eps;
    for (int a = 0; a < 3; ++a) {
        g.extent[a] = (float)cfg.grid_size[a] * cfg.eps;
        g.half[a] = g.extent[a] * 0.5f;
    }
    const float PI_F = 3.14159265358979323846f;
    // smoothing_poly6_normalization / gradient_spiky_normalization kernels.rs:126-140
    if (cfg.dim == 2) {
        g.k6 = 4.0f / (PI_F * host_powi(cfg.eps, 8));
        g.k5 = 10.0f / (PI_F * host_powi(cfg.eps, 5));
    } else {
        g.k6 = 315.0f / (64.0f * PI_F * host_powi(cfg.eps, 9));
        g.k5 = 15.0f / (PI_F * host_powi(cfg.eps, 6));
    }
    return g;
}

bool make_plan(const npa_grid_cfg& cfg, uint32_t batch, uint32_t n, HashgridPlan* plan,
               std::string* err, uint32_t tpi) {
    uint64_t cells = 1;
    for (uint32_t a = 0; a < cfg.dim; ++a) cells *= cfg.grid_size[a];
    if (cells > 65536) {
        *err = "device hashgrid supports at most 65536 cells per system, got " + std::to_string(cells);
        return false;
    }
    const uint64_t total = (uint64_t)batch * n;
    if (total >= (1ull << 31) || (uint64_t)batch * cells + 1 >= (1ull << 32)) {
        *err = "batch_size * particle_count and batch_size * cell_count must stay below 2^31";
        return false;
    }
    HashgridPlan p;
    p.cells = (uint32_t)cells;
    p.key_bits = cells <= 1 ? 0 : 32 - __builtin_clz((uint32_t)cells - 1);
    // ranking waves per tile: one LDS counter row (2 bytes per cell) each, up to 128 KiB of rows;
    // a 1024-thread block (4,096 or more cells) ranks with up to all 16 of its waves, one round each
    // where the tile budget allows, instead of four waves walking four rounds in turn
    p.waves = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(cells >= 4096 ? 16 : 4, 65536 / cells));
    p.lds_bytes = p.waves * p.cells * 2;
    // table entries allowed: 4 per particle, or 64 rows of cells when the cells outnumber the
    // particles (sparse grids: more, smaller tiles keep the O(cells) work per tile parallel)
    const uint64_t budget = std::max<uint64_t>(4 * (uint64_t)n, cells > n ? 64 * cells : cells);
    uint32_t rounds = 1;
    while (rounds < 32) {
        uint64_t tile = (uint64_t)p.waves * rounds * 64;
        uint64_t tiles = (n + tile - 1) / tile;
        if (tiles * cells <= budget) break;
        rounds *= 2;
    }
    p.rounds = rounds;
    p.tile = p.waves * rounds * 64;
    p.tiles_per_sys = std::max<uint32_t>(1, (n + p.tile - 1) / p.tile);
    p.table_entries = (uint64_t)batch * p.tiles_per_sys * cells;
    if (p.table_entries >= (1ull << 32)) {
        *err = "hashgrid tile table exceeds 2^32 entries";
        return false;
    }
    p.tpi = tpi;
    // items: <= tpi slots of one cell run (or of an unsplit bin), so at most total / tpi full
    // items plus one partial item per run
    p.worklist_cap = (total + tpi - 1) / tpi + std::min<uint64_t>(total, (uint64_t)batch * cells * kDirGroups) + 1;
    *plan = p;
    return true;
}

// A wave's LDS counter row, read and written by different lanes in turn: volatile, and in the LDS
// address space (a volatile access through a generic pointer compiles to a flat access, which
// waits on the vector memory counter).
typedef volatile __attribute__((address_space(3))) uint16_t lds_u16;

// The lanes of `peers` whose key equals this lane's in bits [0, key_bits): one ballot per bit,
// keeping the lanes whose bit matches (t = 0 or ~0 is this lane's bit).
__device__ __forceinline__ uint64_t match_key_bits(uint64_t peers, uint32_t key, uint32_t key_bits) {
    uint32_t lo = (uint32_t)peers, hi = (uint32_t)(peers >> 32);
    for (uint32_t bit = 0; bit < key_bits; ++bit) {
        const uint32_t t = (uint32_t)((int32_t)(key << (31u - bit)) >> 31);
        const uint64_t m = __ballot(t != 0u);
        lo &= ~((uint32_t)m ^ t);
        hi &= ~((uint32_t)(m >> 32) ^ t);
    }
    return ((uint64_t)hi << 32) | lo;
}

// ---------------------------------------------------------------- kernels
// keys_in == nullptr: keys are the cells of `pos` (hashgrid build); otherwise the keys
// are read from keys_in and the item count from *d_count (a device-resident count
// bounded by the tiles the grid covers).
template <int R>
__global__ __launch_bounds__(1024) void k_hash_rank(const float4* __restrict__ pos,
                                                   const uint32_t* __restrict__ keys_in,
                                                   const uint32_t* __restrict__ d_count, uint32_t n,
                                                   uint32_t tiles_per_sys, uint32_t waves,
                                                   GridParams g, uint32_t key_bits,
                                                   uint32_t* __restrict__ keys,
                                                   uint32_t* __restrict__ ranks,
                                                   uint32_t* __restrict__ table,
                                                   uint32_t* __restrict__ flags,
                                                   uint32_t* __restrict__ wl_count,
                                                   unsigned long long* __restrict__ scan_status,
                                                   uint32_t nstatus, SplitTargets T,
                                                   int* __restrict__ tile_span, uint32_t pack) {
    extern __shared__ uint16_t cnt[];
    __shared__ int span_red[6][16];
    const uint32_t C = g.cells;
    // folded build (tile_span set): the tile's update-mask targets per key are counted too (u16
    // pairs after the rank counters) and go to the table's high half, and the tile's cell
    // coordinate span goes to tile_span[tile] (min x, y, z, max x, y, z). With pack (a wave ranks at
    // most 128 particles, R <= 2) each wave's counter holds its count in the low byte and its
    // targets in the high byte, so a target also gets its rank among the tile's targets of its key
    // (ranks[i] = rank | target rank << 16) and no target counters are needed.
    const bool fold = tile_span != nullptr;
    uint32_t* mcnt = reinterpret_cast<uint32_t*>(cnt + ((waves * C + 1) & ~1u));
    const uint32_t tile = blockIdx.x;
    const uint32_t b = tile / tiles_per_sys;
    const uint32_t t = tile - b * tiles_per_sys;
    const uint64_t sys_start = (uint64_t)b * n;
    if (d_count) {
        const uint32_t dc = *d_count;
        n = dc < n ? dc : n;
    }
    const uint32_t nwords = waves * C;
    for (uint32_t k = threadIdx.x; k < nwords / 8; k += blockDim.x) reinterpret_cast<uint4*>(cnt)[k] = make_uint4(0, 0, 0, 0);
    for (uint32_t k = nwords / 8 * 8 + threadIdx.x; k < nwords; k += blockDim.x) cnt[k] = 0;
    if (fold && !pack)
        for (uint32_t k = threadIdx.x; k < (C + 1) / 2; k += blockDim.x) mcnt[k] = 0u;
    if (wl_count && tile == 0)  // work-list counters and item queues
        for (uint32_t k = threadIdx.x; k < kWlWords; k += blockDim.x) wl_count[k] = 0;
    for (uint32_t k = tile * blockDim.x + threadIdx.x; k < nstatus; k += gridDim.x * blockDim.x)
        scan_status[k] = 0ull;  // the one-pass offsets scan's published totals (see k_table_offsets_scan)
    // every round's key first, while the counters' clear completes: the position loads and the cell
    // coordinates overlap the clear and the barrier (the keys touch no LDS)
    // The first `waves` waves rank (one LDS counter row each); every wave of the block clears the
    // counters and writes the histogram row, which costs O(C) whatever the tile size.
    const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool ranker = w < waves;
    lds_u16* mine = (lds_u16*)(cnt + (ranker ? w : 0) * C);
    const uint32_t wave_start = t * (waves * R * 64) + w * (R * 64);
    const uint64_t lt = lanemask_lt();
    uint32_t key_r[R], rank_r[R];
#pragma unroll
    for (int r = 0; r < R; ++r) key_r[r] = rank_r[r] = 0;
    bool ovf = false;
    int lo[3] = {INT32_MAX, INT32_MAX, INT32_MAX}, hi[3] = {INT32_MIN, INT32_MIN, INT32_MIN};
    uint32_t tgt_bits = 0;
    if (ranker) {
    // every round's key first (all of the wave's loads in flight together), then the rounds' ranks
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = wave_start + r * 64 + lane;
        const uint64_t at = sys_start + (li < n ? li : 0u);  // (a tile has a particle whenever n > 0)
        if (n == 0) {
            key_r[r] = 0;
        } else if (keys_in) {
            key_r[r] = keys_in[at];
        } else {
            const float4 p4 = pos[at];
            float p[4] = {p4.x, p4.y, p4.z, p4.w};
            int64_t c[3];
            bool o = false;
            cell_coords(p, g, c, &o);
            key_r[r] = cell_of_coords(c, g);
            ovf = ovf || (o && li < n);
            if (fold && li < n) {
#pragma unroll
                for (int a = 0; a < 3; ++a) {
                    const int v = (int)(c[a] < INT32_MIN ? INT32_MIN : (c[a] > INT32_MAX ? INT32_MAX : c[a]));
                    lo[a] = min(lo[a], v);
                    hi[a] = max(hi[a], v);
                }
                const bool tgt = T.mask_mode == 0 ||
                                 (T.mask_mode == 1 ? hash_mask(li, b, n, T.update_prob, T.step_index, T.base_seed)
                                                   : T.mask[at]) != 0.0f;
                if (tgt) tgt_bits |= 1u << r;
            }
        }
    }
    }
    __syncthreads();
    if (ranker) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = wave_start + r * 64 + lane;
        const bool active = li < n;
        const uint32_t key = active ? key_r[r] : 0u;
        uint64_t peers = __ballot(active);
        peers = match_key_bits(peers, key, key_bits);
        const uint64_t tball = fold ? __ballot(active && ((tgt_bits >> r) & 1u)) : 0ull;
        uint32_t rank = 0;
        if (active) {
            const uint32_t below = (uint32_t)__popcll(peers & lt);
            const uint32_t base = mine[key];
            if (pack) {
                rank = (base & 0xffu) + below;
                rank |= ((base >> 8) + (uint32_t)__popcll(peers & tball & lt)) << 16;
                if ((peers >> lane) == 1ull)
                    mine[key] = (uint16_t)(base + (uint32_t)__popcll(peers) + ((uint32_t)__popcll(peers & tball) << 8));
            } else {
                rank = base + below;
                if ((peers >> lane) == 1ull) {
                    mine[key] = (uint16_t)(base + (uint32_t)__popcll(peers));
                    const uint32_t m = (uint32_t)__popcll(peers & tball);
                    if (m) atomicAdd(&mcnt[key >> 1], m << (16 * (key & 1u)));
                }
            }
        }
        key_r[r] = key;
        rank_r[r] = rank;
    }
    }
    if (fold) {  // the tile's coordinate span
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const int l = wave_min_i32(lo[a]), h = wave_max_i32(hi[a]);
            if (lane == 0) {
                span_red[a][w] = l;
                span_red[3 + a][w] = h;
            }
        }
    }
    __syncthreads();
    if (fold && threadIdx.x < 6) {
        const bool is_lo = threadIdx.x < 3;
        int v = is_lo ? INT32_MAX : INT32_MIN;
        for (uint32_t w2 = 0; w2 < blockDim.x / 64; ++w2) v = is_lo ? min(v, span_red[threadIdx.x][w2]) : max(v, span_red[threadIdx.x][w2]);
        tile_span[(uint64_t)tile * 8 + threadIdx.x] = v;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = wave_start + r * 64 + lane;
        if (ranker && li < n) {
            uint32_t prefix = 0;
            if (pack) {  // the earlier waves' counts and targets, field by field
                uint32_t pt = 0;
                for (uint32_t w2 = 0; w2 < w; ++w2) {
                    const uint32_t v = cnt[w2 * C + key_r[r]];
                    prefix += v & 0xffu;
                    pt += v >> 8;
                }
                prefix |= pt << 16;
            } else {
                for (uint32_t w2 = 0; w2 < w; ++w2) prefix += cnt[w2 * C + key_r[r]];
            }
            if (!keys_in) keys[sys_start + li] = key_r[r];
            ranks[sys_start + li] = prefix + rank_r[r];
        }
    }
    uint32_t* row = table + (uint64_t)tile * C;
    if (pack && (C & 3u) == 0) {
        // four consecutive keys per thread: one 8-byte LDS read per wave row and one 16-byte store
        // (C % 4 == 0 keeps every wave row's keys 8-byte aligned)
        for (uint32_t k4 = 4 * threadIdx.x; k4 < C; k4 += 4 * blockDim.x) {
            uint32_t c01 = 0, c23 = 0, t01 = 0, t23 = 0;  // counts and targets, two keys per word
            for (uint32_t w2 = 0; w2 < waves; ++w2) {
                const uint2 v = *reinterpret_cast<const uint2*>(cnt + w2 * C + k4);
                // each u16: count in the low byte, targets in the high byte
                c01 += v.x & 0x00ff00ffu;
                t01 += (v.x >> 8) & 0x00ff00ffu;
                c23 += v.y & 0x00ff00ffu;
                t23 += (v.y >> 8) & 0x00ff00ffu;
            }
            *reinterpret_cast<uint4*>(row + k4) =
                make_uint4((c01 & 0xffffu) | ((t01 & 0xffffu) << 16), (c01 >> 16) | ((t01 >> 16) << 16),
                           (c23 & 0xffffu) | ((t23 & 0xffffu) << 16), (c23 >> 16) | ((t23 >> 16) << 16));
        }
    } else if ((C & 3u) == 0) {
        // the same shape with whole u16 counts (a wave counts at most 256 particles, so each 16-bit
        // half of a sum stays below 2^16); folded: the targets from the u16 pairs after the counters
        for (uint32_t k4 = 4 * threadIdx.x; k4 < C; k4 += 4 * blockDim.x) {
            uint32_t c01 = 0, c23 = 0;
            for (uint32_t w2 = 0; w2 < waves; ++w2) {
                const uint2 v = *reinterpret_cast<const uint2*>(cnt + w2 * C + k4);
                c01 += v.x;
                c23 += v.y;
            }
            uint4 o = make_uint4(c01 & 0xffffu, c01 >> 16, c23 & 0xffffu, c23 >> 16);
            if (fold) {
                const uint2 mm = *reinterpret_cast<const uint2*>(mcnt + (k4 >> 1));
                o.x |= (mm.x & 0xffffu) << 16;
                o.y |= (mm.x >> 16) << 16;
                o.z |= (mm.y & 0xffffu) << 16;
                o.w |= (mm.y >> 16) << 16;
            }
            *reinterpret_cast<uint4*>(row + k4) = o;
        }
    } else
    for (uint32_t k = threadIdx.x; k < C; k += blockDim.x) {
        uint32_t tot = 0;
        if (pack) {
            uint32_t tt = 0;
            for (uint32_t w2 = 0; w2 < waves; ++w2) {
                const uint32_t v = cnt[w2 * C + k];
                tot += v & 0xffu;
                tt += v >> 8;
            }
            tot |= tt << 16;
        } else {
            for (uint32_t w2 = 0; w2 < waves; ++w2) tot += cnt[w2 * C + k];
            // folded: the tile's targets of the key in the high half (a tile holds at most 32,768)
            if (fold) tot |= ((mcnt[k >> 1] >> (16 * (k & 1u))) & 0xffffu) << 16;
        }
        row[k] = tot;
    }
    if (ovf) atomicOr(flags, 1u);
}

// A key's column of the tile table (tiles entries C apart) -> exclusive per-tile bases; returns
// the column's total. Every load of a batch is issued before its first store: the round trips,
// not the loads, set the scans' time (C2, 64 tiles: 6.9 us in batches of 8, 4.9 us in batches
// of 32).
__device__ __forceinline__ uint32_t column_scan(uint32_t* __restrict__ col, uint32_t C, uint32_t tiles) {
    uint32_t run = 0, t = 0;
    for (; t + 32 <= tiles; t += 32) {
        uint32_t v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = col[(uint64_t)(t + u) * C];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            col[(uint64_t)(t + u) * C] = run;
            run += v[u];
        }
    }
    for (; t + 8 <= tiles; t += 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = col[(uint64_t)(t + u) * C];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            col[(uint64_t)(t + u) * C] = run;
            run += v[u];
        }
    }
    for (; t < tiles; ++t) {
        const uint32_t v = col[(uint64_t)t * C];
        col[(uint64_t)t * C] = run;
        run += v;
    }
    return run;
}

__global__ __launch_bounds__(256) void k_table_scan(uint32_t* __restrict__ table,
                                                    uint32_t* __restrict__ totals, uint32_t C,
                                                    uint32_t tiles_per_sys) {
    const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (k >= C) return;
    totals[(uint64_t)b * C + k] = column_scan(table + (uint64_t)b * tiles_per_sys * C + k, C, tiles_per_sys);
}

// The column scan and the offsets scan in one pass, for the hashgrid build. A block's position
// comes from a ticket (status[gridDim.x * gridDim.y], an atomic counter), not from its block index:
// ticket q is block x = q mod gridDim.x of system b = q / gridDim.x. Thread k of that block (key
// k = 256 x + thread): table[t][k] -> exclusive per-tile bases, as k_table_scan, and the key's
// total. The block publishes the sum of its keys' totals (bit 63 marks it published; k_hash_rank
// zeroed every status word of this build and the ticket counter), adds the totals published by the
// system's earlier blocks - which took smaller tickets, so they are already running whatever order
// the hardware dispatches blocks in, each of them publishes and the wait ends - and writes
// bin_offsets[b][k] = b * n + its keys' exclusive prefix. The last block of the last system also
// writes the closing entry bin_offsets[batch * C].
__global__ __launch_bounds__(256) void k_table_offsets_scan(uint32_t* __restrict__ table,
                                                            uint32_t* __restrict__ bin_offsets,
                                                            unsigned long long* __restrict__ status, uint32_t C,
                                                            uint32_t tiles_per_sys, uint32_t n, uint32_t batch) {
    __shared__ uint32_t wsum[4];
    __shared__ uint32_t s_prefix, s_ticket;
    if (threadIdx.x == 0)
        s_ticket = (uint32_t)atomicAdd(status + (uint64_t)gridDim.x * gridDim.y, 1ull);
    __syncthreads();
    const uint32_t ticket = s_ticket;
    const uint32_t bx = ticket % gridDim.x;
    const uint32_t k = bx * 256 + threadIdx.x;
    const uint32_t b = ticket / gridDim.x;
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t run = 0;
    if (k < C) {
        run = column_scan(table + (uint64_t)b * tiles_per_sys * C + k, C, tiles_per_sys);
    }
    // the keys' exclusive prefix within the block
    const uint32_t x = wave_incl_add(run);
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    uint32_t wpre = 0, btotal = 0;
#pragma unroll
    for (uint32_t v = 0; v < 4; ++v) {
        if (v < w) wpre += wsum[v];
        btotal += wsum[v];
    }
    const uint64_t row = (uint64_t)b * gridDim.x;
    if (threadIdx.x == 0)
        __hip_atomic_store(status + row + bx, (1ull << 63) | btotal, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    if (w == 0) {  // the system's earlier blocks' totals, 64 at a time
        uint32_t acc = 0;
        for (uint32_t base = 0; base < bx; base += 64) {
            const uint32_t j = base + lane;
            if (j < bx) {
                unsigned long long v;
                do {
                    v = __hip_atomic_load(status + row + j, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                } while (!(v >> 63));
                acc += (uint32_t)v;
            }
        }
        acc = wave_sum_u32(acc);
        if (lane == 0) s_prefix = acc;
    }
    __syncthreads();
    const uint32_t prefix = s_prefix;
    if (k < C) bin_offsets[(uint64_t)b * C + k] = b * n + prefix + wpre + x - run;
    if (b == batch - 1 && bx == gridDim.x - 1 && threadIdx.x == 0)
        bin_offsets[(uint64_t)batch * C] = b * n + prefix + btotal;
}

// The column scan of a folded table (count in the low half, the tile's update-mask targets in the
// high half): per-tile count bases written back as full words; returns the count total and sets
// *masked to the key's targets.
__device__ __forceinline__ uint32_t column_scan_fold(uint32_t* __restrict__ col, uint32_t C, uint32_t tiles,
                                                     uint32_t* masked, uint32_t pack) {
    uint32_t run = 0, mrun = 0, t = 0;
    for (; t + 32 <= tiles; t += 32) {
        uint32_t v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = col[(uint64_t)(t + u) * C];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            col[(uint64_t)(t + u) * C] = pack ? run | (mrun << 16) : run;
            run += v[u] & 0xffffu;
            mrun += v[u] >> 16;
        }
    }
    for (; t + 8 <= tiles; t += 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = col[(uint64_t)(t + u) * C];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            col[(uint64_t)(t + u) * C] = pack ? run | (mrun << 16) : run;
            run += v[u] & 0xffffu;
            mrun += v[u] >> 16;
        }
    }
    for (; t < tiles; ++t) {
        const uint32_t v = col[(uint64_t)t * C];
        col[(uint64_t)t * C] = pack ? run | (mrun << 16) : run;
        run += v & 0xffffu;
        mrun += v >> 16;
    }
    *masked = mrun;
    return run;
}

// The folded build's scan (one system): k_table_offsets_scan's column scan and offsets scan, and
// with them what the split would emit per bin - the first work item of each key (ceil(count / tpi)
// items of <= tpi slots, the split's items for a bin of one cell or an unsplit bin; item_base) and
// its first compact row (row_next, the scatter's per-key row counter), the totals (wl_count[0] and
// [1]) and the directory sizes: one run per occupied bin, or kDirGroups + 1 (unsplit, walked in the
// reference order with the cell filter) for a bin that may hold several cells (the system's cell
// coordinates reach two cells of the bin's residues). Blocks take their position
// from a ticket and publish two status words (count; items | rows << 31) for the look-back, as in
// k_table_offsets_scan.
__global__ __launch_bounds__(256) void k_table_offsets_fold(uint32_t* __restrict__ table,
                                                            uint32_t* __restrict__ bin_offsets,
                                                            unsigned long long* __restrict__ status, uint32_t C,
                                                            uint32_t tiles, uint32_t n, uint32_t tpi_log2, GridParams g,
                                                            const int* __restrict__ tile_span,
                                                            uint32_t* __restrict__ item_base,
                                                            uint32_t* __restrict__ row_next,
                                                            uint32_t* __restrict__ dir_n,
                                                            uint32_t* __restrict__ wl_count, uint32_t pack) {
    __shared__ uint32_t wsum[3][4];
    __shared__ int span[6][4];
    __shared__ uint32_t s_pa, s_pb, s_pm, s_ticket;
    const uint32_t nb = gridDim.x;
    if (threadIdx.x == 0) s_ticket = (uint32_t)atomicAdd(status + 2ull * nb, 1ull);
    __syncthreads();
    const uint32_t bx = s_ticket;
    const uint32_t k = bx * 256 + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t run = 0, msk = 0;
    if (k < C) run = column_scan_fold(table + k, C, tiles, &msk, pack);
    const uint32_t itm = (run + (1u << tpi_log2) - 1) >> tpi_log2;
    // the system's cell coordinate span (Particle mode)
    int lo[3] = {INT32_MAX, INT32_MAX, INT32_MAX}, hi[3] = {INT32_MIN, INT32_MIN, INT32_MIN};
    if (g.mode == 1)
        for (uint32_t t = threadIdx.x; t < tiles; t += 256)
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                lo[a] = min(lo[a], tile_span[(uint64_t)t * 8 + a]);
                hi[a] = max(hi[a], tile_span[(uint64_t)t * 8 + 3 + a]);
            }
    const uint32_t xa = wave_incl_add(run), xb = wave_incl_add(itm), xm = wave_incl_add(msk);
    if (g.mode == 1)
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            lo[a] = wave_min_i32(lo[a]);
            hi[a] = wave_max_i32(hi[a]);
        }
    if (lane == 63) {
        wsum[0][w] = xa;
        wsum[1][w] = xb;
        wsum[2][w] = xm;
    }
    if (lane == 0)
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            span[a][w] = lo[a];
            span[3 + a][w] = hi[a];
        }
    __syncthreads();
    uint32_t pa = 0, pb = 0, pm = 0, ta = 0, tb = 0, tm = 0;
#pragma unroll
    for (uint32_t v = 0; v < 4; ++v) {
        if (v < w) {
            pa += wsum[0][v];
            pb += wsum[1][v];
            pm += wsum[2][v];
        }
        ta += wsum[0][v];
        tb += wsum[1][v];
        tm += wsum[2][v];
    }
    // A coordinate bin (residues r_a = c_a mod size_a) can hold two cells only if on some axis two
    // coordinates of the system's span [lo, hi] share its residue: first = lo + ((r - lo) mod size)
    // and first + size <= hi. Such bins are marked unsplit (walked with the cell filter, exact for
    // any bin); every other occupied bin holds one cell.
    bool alias = false;
    int sl[3], sh[3];
    bool wide = false;  // some axis of the span wider than the grid (block-uniform)
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        sl[a] = INT32_MAX;
        sh[a] = INT32_MIN;
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v) {
            sl[a] = min(sl[a], span[a][v]);
            sh[a] = max(sh[a], span[3 + a][v]);
        }
        if (a < g.dim && sh[a] >= sl[a] && (int64_t)sh[a] - (int64_t)sl[a] >= (int64_t)g.size[a]) wide = true;
    }
    if (g.mode == 1 && wide && k < C && run) {
        uint32_t rest = k;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            if (a < g.dim) {
                const int64_t m = (int64_t)g.size[a];
                const int64_t r = (int64_t)(rest % g.size[a]);
                rest /= g.size[a];
                const int64_t l = sl[a], h = sh[a];
                if (h >= l && h - l >= m && l + rem_euclid_i64(r - l, m) + m <= h) alias = true;
            }
        }
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(status + bx, (1ull << 63) | ta, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(status + nb + bx, (1ull << 63) | tb | ((unsigned long long)tm << 31), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (w == 0) {  // the earlier blocks' totals, 64 at a time (they took smaller tickets: running)
        uint32_t acc_a = 0, acc_b = 0, acc_m = 0;
        for (uint32_t base = 0; base < bx; base += 64) {
            const uint32_t j = base + lane;
            if (j < bx) {
                unsigned long long v, u;
                do {
                    v = __hip_atomic_load(status + j, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                } while (!(v >> 63));
                do {
                    u = __hip_atomic_load(status + nb + j, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                } while (!(u >> 63));
                acc_a += (uint32_t)v;
                acc_b += (uint32_t)(u & 0x7fffffffull);
                acc_m += (uint32_t)((u >> 31) & 0x7fffffffull);
            }
        }
        acc_a = wave_sum_u32(acc_a);
        acc_b = wave_sum_u32(acc_b);
        acc_m = wave_sum_u32(acc_m);
        if (lane == 0) {
            s_pa = acc_a;
            s_pb = acc_b;
            s_pm = acc_m;
        }
    }
    __syncthreads();
    if (k < C) {
        bin_offsets[k] = s_pa + pa + xa - run;
        item_base[k] = s_pb + pb + xb - itm;
        row_next[k] = s_pm + pm + xm - msk;
        if (g.mode == 1) dir_n[k] = run ? (alias ? kDirGroups + 1 : 1u) : 0u;
    }
    if (bx == nb - 1 && threadIdx.x == 0) {
        bin_offsets[C] = s_pa + ta;
        wl_count[0] = s_pb + tb;
        wl_count[1] = s_pm + tm;
    }
}

// Exclusive scan of one value per thread over a 1024-thread block.
__device__ __forceinline__ uint32_t block_scan_1024(uint32_t v, uint32_t* lds, uint32_t* total);

// The same two scans for many small systems (batched rollouts): one 1024-thread block per system,
// thread t owning keys [t PER, t PER + PER) (C <= 1024 PER) over TL tiles (tiles_per_sys <= TL). All
// of a thread's table entries are loaded at once; each key's column becomes its exclusive per-tile
// bases, and one block scan of the threads' totals gives bin_offsets[b][k] = b * n + the key's
// exclusive prefix. No block waits for another (the one-pass kernel's look-back polls the other
// blocks' published totals, which costs more than it saves when thousands of blocks poll at once).
template <int PER, int TL>
__global__ __launch_bounds__(1024) void k_table_offsets_sys(uint32_t* __restrict__ table,
                                                          uint32_t* __restrict__ bin_offsets, uint32_t C,
                                                          uint32_t tiles_per_sys, uint32_t n, uint32_t batch) {
    __shared__ uint32_t lds[16];
    const uint32_t b = blockIdx.x;
    const uint32_t k0 = threadIdx.x * PER;
    uint32_t* tab = table + (uint64_t)b * tiles_per_sys * C;
    uint32_t v[PER][TL];
#pragma unroll
    for (int q = 0; q < PER; ++q)
#pragma unroll
        for (int t = 0; t < TL; ++t)
            v[q][t] = k0 + q < C && (uint32_t)t < tiles_per_sys ? tab[(uint64_t)t * C + k0 + q] : 0u;
    uint32_t tot[PER], sum = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        uint32_t run = 0;
#pragma unroll
        for (int t = 0; t < TL; ++t) {
            if (k0 + q < C && (uint32_t)t < tiles_per_sys) tab[(uint64_t)t * C + k0 + q] = run;
            run += v[q][t];
        }
        tot[q] = run;
        sum += run;
    }
    uint32_t all;
    uint32_t pre = block_scan_1024(sum, lds, &all);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        if (k0 + q < C) bin_offsets[(uint64_t)b * C + k0 + q] = b * n + pre;
        pre += tot[q];
    }
    if (b == batch - 1 && threadIdx.x == 0) bin_offsets[(uint64_t)batch * C] = b * n + all;
}

__device__ __forceinline__ uint32_t block_scan_1024(uint32_t v, uint32_t* lds, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t x = wave_incl_add(v);
    if (lane == 63) lds[wid] = x;
    __syncthreads();
    if (wid == 0) {
        const uint32_t s = wave_incl_add(lane < nw ? lds[lane] : 0u);
        if (lane < nw) lds[lane] = s;
    }
    __syncthreads();
    const uint32_t wave_prefix = wid ? lds[wid - 1] : 0;
    *total = lds[nw - 1];
    __syncthreads();
    return wave_prefix + x - v;
}

// One block per system: bin_offsets[b][k] = b * n + exclusive prefix of totals[b][k] over k.
// Thread t owns the PER consecutive keys [t PER, t PER + PER) (C <= 1024 PER): all of its loads are
// issued at once (16-byte loads when the rows are aligned), one block scan orders the threads, and
// the prefixes are written with a running carry - one load, one scan and one store whatever C.
template <int PER>
__global__ __launch_bounds__(1024) void k_offsets_scan(const uint32_t* __restrict__ totals,
                                                       uint32_t* __restrict__ bin_offsets,
                                                       uint32_t C, uint32_t n, uint32_t batch) {
    __shared__ uint32_t lds[16];
    const uint32_t b = blockIdx.x;
    const uint32_t* tot = totals + (uint64_t)b * C;
    uint32_t* out = bin_offsets + (uint64_t)b * C;
    const uint32_t k0 = threadIdx.x * PER;
    uint32_t v[PER];
    const bool vec = PER % 4 == 0 && ((uint64_t)b * C) % 4 == 0 && k0 + PER <= C;
    if (vec) {
#pragma unroll
        for (int j = 0; j < PER; j += 4) {
            const uint4 q = *reinterpret_cast<const uint4*>(tot + k0 + j);
            v[j] = q.x;
            v[j + 1] = q.y;
            v[j + 2] = q.z;
            v[j + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) v[j] = k0 + j < C ? tot[k0 + j] : 0u;
    }
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) sum += v[j];
    uint32_t all;
    uint32_t run = b * n + block_scan_1024(sum, lds, &all);
    if (vec) {
#pragma unroll
        for (int j = 0; j < PER; j += 4) {
            uint4 q;
            q.x = run;
            run += v[j];
            q.y = run;
            run += v[j + 1];
            q.z = run;
            run += v[j + 2];
            q.w = run;
            run += v[j + 3];
            *reinterpret_cast<uint4*>(out + k0 + j) = q;
        }
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            if (k0 + j < C) out[k0 + j] = run;
            run += v[j];
        }
    }
    // last entry = total count (every system holds n entries when the counts are per system)
    if (b == batch - 1 && threadIdx.x == 0) bin_offsets[(uint64_t)batch * C] = b * n + all;
}

// k_offsets_scan with the smallest PER that covers C (<= 65536) keys.
static hipError_t launch_offsets_scan(const uint32_t* totals, uint32_t* bin_offsets, uint32_t C, uint32_t n,
                                      uint32_t batch, hipStream_t stream, Profiler* prof) {
    const uint32_t per = (C + 1023) / 1024;
    auto launch = [&](auto k) {
        return launch_timed(prof, NPA_KERNEL_OFFSETS_SCAN, k, dim3(batch), dim3(1024), 0, stream, totals,
                            bin_offsets, C, n, batch);
    };
    if (per <= 1) return launch(k_offsets_scan<1>);
    if (per <= 4) return launch(k_offsets_scan<4>);
    if (per <= 8) return launch(k_offsets_scan<8>);
    if (per <= 16) return launch(k_offsets_scan<16>);
    if (per <= 32) return launch(k_offsets_scan<32>);
    return launch(k_offsets_scan<64>);
}

// The reference's snapshot only: perm (slot -> particle of the system) and inv. (The rollout step
// scatters its whole sorted payload with k_scatter_payload.)
__global__ __launch_bounds__(256) void k_scatter(uint32_t n, uint32_t total, uint32_t tile,
                                                 uint32_t tiles_per_sys, uint32_t C,
                                                 const uint32_t* __restrict__ keys,
                                                 const uint32_t* __restrict__ ranks,
                                                 const uint32_t* __restrict__ table,
                                                 const uint32_t* __restrict__ bin_offsets,
                                                 uint32_t* __restrict__ out, uint32_t* __restrict__ inv,
                                                 uint32_t* __restrict__ flags) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    // This build's coordinate-overflow flag (set by k_hash_rank, which has finished) moves into the
    // sticky word the synchronising entry points report, so the next build starts clean.
    if (i == 0) {
        const uint32_t f = flags[0];
        if (f) {
            flags[1] |= f;
            flags[0] = 0;
        }
    }
    if (i >= total) return;
    const uint32_t b = i / n;
    const uint32_t li = i - b * n;
    const uint32_t t = li / tile;
    const uint32_t key = keys[i];
    const uint32_t dst_local = (bin_offsets[(uint64_t)b * C + key] - b * n) +
                               table[((uint64_t)b * tiles_per_sys + t) * C + key] + ranks[i];
    const uint32_t dst = b * n + dst_local;
    out[dst] = li;
    inv[i] = dst_local;
}

// The folded build's per-particle outputs (item_base null: not folding): the split's compact rows,
// work items and directory entries, written by the payload scatter.
struct FoldOut {
    const uint32_t* item_base = nullptr;  // [C] first work item of each key
    uint32_t* row_next = nullptr;         // [C] next compact row of each key (atomic)
    uint2* worklist = nullptr;
    uint32_t* act_rows = nullptr;
    uint32_t* row_of = nullptr;
    int4* dir_e = nullptr;
    uint32_t tpi_log2 = 0;
    // packed: table entries hold the tile's count | target prefixes << 16 and ranks[i] the rank |
    // target rank << 16, so a target's compact row needs no atomic
    uint32_t packed = 0;
};

// Copies nq (1, 2, 4, 6 or 8) float4s with every load issued before the first store.
template <int NQ>
__device__ __forceinline__ void copy_row4_n(float4* __restrict__ dst, const float4* __restrict__ src) {
    float4 v[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) v[q] = src[q];
#pragma unroll
    for (int q = 0; q < NQ; ++q) dst[q] = v[q];
}
__device__ __forceinline__ void copy_row4(float4* __restrict__ dst, const float4* __restrict__ src, uint32_t nq) {
    switch (nq) {
        case 1: copy_row4_n<1>(dst, src); break;
        case 2: copy_row4_n<2>(dst, src); break;
        case 4: copy_row4_n<4>(dst, src); break;
        case 6: copy_row4_n<6>(dst, src); break;
        default: copy_row4_n<8>(dst, src); break;
    }
}

// Writes particle i (global index) to sorted slot dst: snapshot entries, sorted record
// {x, y, bits(cx), bits(cy)} (2D) or position + coordinates (3D), and the zero-padded state row.
template <int D>
__device__ __forceinline__ void write_sorted(uint32_t dst, uint32_t i, uint32_t b, uint32_t n,
                                             const float4& p4, const int c[3], const float* __restrict__ states,
                                             uint32_t S, uint32_t* __restrict__ perm, uint32_t* __restrict__ inv,
                                             float4* __restrict__ srec, int4* __restrict__ scoord,
                                             float* __restrict__ sstate) {
    perm[dst] = i - b * n;
    inv[i] = dst - b * n;
    if (D == 2) {
        srec[dst] = make_float4(p4.x, p4.y, __int_as_float(c[0]), __int_as_float(c[1]));
    } else {
        srec[dst] = p4;
        scoord[dst] = make_int4(c[0], c[1], c[2], (int)i);
    }
    if (!states) return;  // neighbour-list export needs positions only
    const uint32_t SS = state_stride_for(S);
    const float* src = states + (uint64_t)i * S;
    float4* o4 = reinterpret_cast<float4*>(sstate + (uint64_t)dst * SS);
    if (S == SS) {  // rows are 16-byte aligned (checked on the host)
        copy_row4(o4, reinterpret_cast<const float4*>(src), SS / 4);
    } else {
        for (uint32_t q = 0; q < SS / 4; ++q) {
            const uint32_t cc = 4 * q;
            o4[q] = make_float4(cc < S ? src[cc] : 0.0f, cc + 1 < S ? src[cc + 1] : 0.0f,
                                cc + 2 < S ? src[cc + 2] : 0.0f, cc + 3 < S ? src[cc + 3] : 0.0f);
        }
    }
}

// Payload scatter: every particle writes its sorted record, state row and snapshot entries at its
// slot of the stable counting sort (the reference's order within each bin), and a particle outside
// the step's update mask is written to the step's output here (hold_particle). k_split keeps this
// payload for a bin that holds one cell, or more cells than its directory holds (both stay in the
// reference order), and rewrites the bins whose cells it reorders. out[slot] = global particle index.
template <int D>
__global__ __launch_bounds__(256) void k_scatter_payload(uint32_t n, uint32_t total, uint32_t tile,
                                                         uint32_t tiles_per_sys, uint32_t C,
                                                         const uint32_t* __restrict__ keys,
                                                         const uint32_t* __restrict__ ranks,
                                                         const uint32_t* __restrict__ table,
                                                         const uint32_t* __restrict__ bin_offsets,
                                                         uint32_t* __restrict__ out, uint32_t* __restrict__ perm,
                                                         uint32_t* __restrict__ inv, const float4* __restrict__ pos,
                                                         const float* __restrict__ states, uint32_t S, GridParams g,
                                                         float4* __restrict__ srec, int4* __restrict__ scoord,
                                                         float* __restrict__ sstate, SplitTargets T,
                                                         uint32_t* __restrict__ flags, FoldOut F) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    // this build's coordinate-overflow flag (set by k_hash_rank) moves into the sticky word
    if (i == 0) {
        const uint32_t f = flags[0];
        if (f) {
            flags[1] |= f;
            flags[0] = 0;
        }
    }
    if (i >= total) return;
    const uint32_t b = i / n;
    const uint32_t li = i - b * n;
    const float4 p4 = pos[i];  // independent of the slot: in flight while the slot is computed
    const uint32_t key = keys[i];
    // the update mask's hash needs no load: computed while the loads above are in flight (a mask
    // array's value is loaded with them and tested once the slot is known)
    const float hm = T.mask_mode == 1 ? hash_mask(li, b, n, T.update_prob, T.step_index, T.base_seed) : 1.0f;
    const float am = T.mask_mode == 2 ? T.mask[i] : 1.0f;
    const uint32_t t = li / tile;
    const uint32_t beg = bin_offsets[(uint64_t)b * C + key];
    const uint32_t tv = table[((uint64_t)b * tiles_per_sys + t) * C + key], rv = ranks[i];
    // the cell coordinates need only the position: computed while the slot's words are in flight
    const float p[4] = {p4.x, p4.y, p4.z, p4.w};
    int64_t c64[3];
    bool ovf = false;
    cell_coords(p, g, c64, &ovf);
    const int c[3] = {(int)c64[0], (int)c64[1], (int)c64[2]};
    const uint32_t r_bin = F.packed ? (tv & 0xffffu) + (rv & 0xffffu) : tv + rv;  // rank in the bin
    const uint32_t dst = beg + r_bin;
    if (!F.item_base) out[dst] = i;
    write_sorted<D>(dst, i, b, n, p4, c, states, S, perm, inv, srec, scoord, sstate);
    const bool tgt = T.mask_mode == 0 || (T.mask_mode == 1 ? hm : am) != 0.0f;
    if (!tgt) hold_particle(i, S, g, T.pos, T.states, T.out_pos, T.out_states);
    if (F.item_base) {  // folded build (one system): what the split emits for the particle's bin
        if (tgt) {
            const uint32_t row = F.packed ? F.row_next[key] + (tv >> 16) + (rv >> 16) : atomicAdd(F.row_next + key, 1u);
            F.act_rows[row] = dst;
            F.row_of[dst] = row;
        } else {
            F.row_of[dst] = ~0u;
        }
        const uint32_t tpi = 1u << F.tpi_log2;
        if ((r_bin & (tpi - 1)) == 0) {
            const uint32_t left = bin_offsets[key + 1] - beg - r_bin;
            F.worklist[F.item_base[key] + (r_bin >> F.tpi_log2)] = make_uint2(dst, left < tpi ? left : tpi);
        }
        if (g.mode == 1 && r_bin == 0) F.dir_e[(uint64_t)key * kDirGroups] = make_int4(c[0], c[1], c[2], (int)dst);
    }
}

// Orders each bin by true cell, one wave per bin. Pass 1 finds the bin's distinct cells in order
// of first appearance and their counts (from the scatter's sorted records); pass 2 places each
// particle at run start of its cell + its rank among the earlier particles of that cell, which
// keeps ascending particle index inside every run (the reference's neighbour order). A bin of one
// cell is already in that order, and a bin with more than kDirGroups cells keeps the reference
// order (dir_n = kDirGroups + 1): both keep the scatter's payload; any other bin is rewritten from
// the step's input arrays. Also emits the wave work items of the density pass (<= tpi consecutive
// slots of one run, or of an unsplit bin) and the second pass's targets: the particles of the
// step's update mask get consecutive compact rows (act_rows[row] = slot, in slot order within the
// bin); the scatter has written the others to the step's output (hold_particle).
constexpr uint32_t kSplitWaves = 16;  // bins (waves) per k_split block
constexpr uint32_t kSplitHeld = 3;    // chunks of 64 slots a k_split wave loads at once and keeps

template <int D>
__global__ __launch_bounds__(1024) void k_split(const float4* __restrict__ pos, const float* __restrict__ states,
                                               uint32_t S, uint32_t n, uint32_t nbins, GridParams g,
                                               const uint32_t* __restrict__ bo,
                                               const uint32_t* __restrict__ order,
                                               uint32_t* __restrict__ perm, uint32_t* __restrict__ inv,
                                               float4* __restrict__ srec, int4* __restrict__ scoord,
                                               float* __restrict__ sstate, uint32_t* __restrict__ dir_n,
                                               int4* __restrict__ dir_e, uint2* __restrict__ worklist,
                                               uint32_t* __restrict__ wl_count, uint32_t tpi, SplitTargets T,
                                               uint32_t* __restrict__ act_rows, uint32_t* __restrict__ row_of,
                                               const uint32_t* __restrict__ bin_list,
                                               const uint32_t* __restrict__ bin_count) {
    constexpr uint32_t K = kDirGroups;
    __shared__ uint32_t s_items[kSplitWaves], s_rows[kSplitWaves];
    __shared__ uint32_t s_base, s_rbase;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // every bin in order, or (bin_list) the listed bins - the ones the one-lane pass left
    uint32_t bin = blockIdx.x * kSplitWaves + wave;
    if (bin_list) {
        const uint32_t listed = *bin_count;
        if (blockIdx.x * kSplitWaves >= listed) return;  // the whole block has no bin
        bin = bin < listed ? bin_list[bin] : nbins;
    }
    const bool has_bin = bin < nbins;
    const uint32_t beg = has_bin ? bo[bin] : 0u, end = has_bin ? bo[bin + 1] : 0u;
    const uint32_t b = has_bin ? bin / g.cells : 0u;
    const uint64_t lt = lanemask_lt();
    int gx[K], gy[K], gz[K];
    uint32_t gc[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        gx[k] = gy[k] = gz[k] = 0;
        gc[k] = 0;
    }
    uint32_t gt[K];  // targets per run
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) gt[k] = 0;
    uint32_t ng = 0;
    bool over = false;
    // update-mask target (the second pass and the MLP serve it)
    auto is_target = [&](bool valid, uint32_t i) -> bool {
        if (!valid) return false;
        if (T.mask_mode == 0) return true;
        const uint32_t li = i - b * n;
        const float m = T.mask_mode == 1 ? hash_mask(li, b, n, T.update_prob, T.step_index, T.base_seed) : T.mask[i];
        return m != 0.0f;
    };
    // the particle of slot c0 + lane and its cell from the scatter's sorted record (coalesced; no
    // slot of the bin is rewritten before the last pass)
    auto load_sorted = [&](uint32_t c0, bool& valid, uint32_t& i, int c[3]) {
        const uint32_t slot = c0 + lane;
        valid = slot < end;
        const uint32_t sl = valid ? slot : c0;
        i = order[sl];
        if constexpr (D == 2) {
            const float4 r = srec[sl];
            c[0] = __float_as_int(r.z);
            c[1] = __float_as_int(r.w);
            c[2] = 0;
        } else {
            const int4 cc = scoord[sl];
            c[0] = cc.x;
            c[1] = cc.y;
            c[2] = cc.z;
        }
    };
    // the same from the step's input arrays (a bin that is reordered overwrites its sorted records)
    auto load = [&](uint32_t c0, bool& valid, uint32_t& i, float4& p4, int c[3]) {
        const uint32_t slot = c0 + lane;
        valid = slot < end;
        i = order[valid ? slot : c0];
        p4 = pos[i];
        const float p[4] = {p4.x, p4.y, p4.z, p4.w};
        int64_t c64[3];
        bool ovf = false;
        cell_coords(p, g, c64, &ovf);  // overflow was flagged by the hash pass
        c[0] = (int)c64[0];
        c[1] = (int)c64[1];
        c[2] = (int)c64[2];
    };
    auto group_of = [&](const int c[3]) -> int {
        int gid = -1;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (k < ng && c[0] == gx[k] && c[1] == gy[k] && c[2] == gz[k]) gid = (int)k;
        return gid;
    };
    // the first kSplitHeld chunks (the whole bin for most bins) are loaded together, before any is
    // used, and kept for both passes; a rewritten bin takes its positions and cells from them
    constexpr uint32_t NH = kSplitHeld;
    bool hv[NH], ht[NH];
    uint32_t hi[NH];
    int hc[NH][3];
    float4 hr[NH];
#pragma unroll
    for (uint32_t k = 0; k < NH; ++k) {
        hv[k] = ht[k] = false;
        hi[k] = 0;
        hc[k][0] = hc[k][1] = hc[k][2] = 0;
        hr[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const uint32_t c0 = beg + 64 * k;
        if (c0 < end) {
            const uint32_t slot = c0 + lane;
            hv[k] = slot < end;
            const uint32_t sl = hv[k] ? slot : c0;
            hr[k] = srec[sl];
            if constexpr (D == 2) {
                hi[k] = order[sl];
                hc[k][0] = __float_as_int(hr[k].z);
                hc[k][1] = __float_as_int(hr[k].w);
            } else {
                const int4 cc = scoord[sl];
                hc[k][0] = cc.x;
                hc[k][1] = cc.y;
                hc[k][2] = cc.z;
                hi[k] = (uint32_t)cc.w;
            }
        }
    }
    // first pass over one chunk: new cells join the directory in order of first appearance
    auto count_chunk = [&](bool valid, uint32_t i, const int c[3]) -> bool {
        int gid = group_of(c);
        uint64_t unknown = __ballot(valid && gid < 0);
        while (unknown) {
            if (ng == K) {
                over = true;
                break;
            }
            const int leader = __ffsll((unsigned long long)unknown) - 1;
            const int nx = __builtin_amdgcn_readlane(c[0], leader);
            const int ny = __builtin_amdgcn_readlane(c[1], leader);
            const int nz = __builtin_amdgcn_readlane(c[2], leader);
#pragma unroll
            for (uint32_t k = 0; k < K; ++k)
                if (k == ng) {
                    gx[k] = nx;
                    gy[k] = ny;
                    gz[k] = nz;
                }
            if (valid && gid < 0 && c[0] == nx && c[1] == ny && c[2] == nz) gid = (int)ng;
            ++ng;
            unknown = __ballot(valid && gid < 0);
        }
        const bool tgt = is_target(valid, i);
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            gc[k] += (uint32_t)__popcll(__ballot(valid && gid == (int)k));
            gt[k] += (uint32_t)__popcll(__ballot(tgt && gid == (int)k));
        }
        return tgt;
    };
#pragma unroll
    for (uint32_t k = 0; k < NH; ++k)
        if (beg + 64 * k < end && !over) ht[k] = count_chunk(hv[k], hi[k], hc[k]);
    for (uint32_t c0 = beg + 64 * NH; c0 < end && !over; c0 += 64) {
        bool valid;
        uint32_t i;
        int c[3];
        load_sorted(c0, valid, i, c);
        count_chunk(valid, i, c);
    }
    uint32_t nitems = 0, nrows = 0;
    uint32_t start[K];
    if (over) {  // one run in the reference order: count its targets
        nitems = (end - beg + tpi - 1) / tpi;
        for (uint32_t c0 = beg; c0 < end; c0 += 64) {
            const uint32_t slot = c0 + lane;
            const bool valid = slot < end;
            nrows += (uint32_t)__popcll(__ballot(is_target(valid, order[valid ? slot : c0])));
        }
    } else {
        uint32_t run = beg;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            start[k] = run;
            run += gc[k];
            nitems += (gc[k] + tpi - 1) / tpi;
            nrows += gt[k];
        }
    }
    // one work-list and one row reservation per block: the waves' counts are summed in LDS
    if (lane == 0) {
        s_items[wave] = nitems;
        s_rows[wave] = nrows;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t tot = 0, rows = 0;
        for (uint32_t w = 0; w < kSplitWaves; ++w) {
            tot += s_items[w];
            rows += s_rows[w];
        }
        // items (low word) and rows (high word) reserved by one atomic
        const unsigned long long add = (unsigned long long)tot | ((unsigned long long)rows << 32);
        const unsigned long long old = add ? atomicAdd(reinterpret_cast<unsigned long long*>(wl_count), add) : 0ull;
        s_base = (uint32_t)old;
        s_rbase = (uint32_t)(old >> 32);
    }
    __syncthreads();
    uint32_t wbase = s_base;  // first work item of this bin
    uint32_t rbase = s_rbase;  // first compact row of this bin
    for (uint32_t w = 0; w < wave; ++w) {
        wbase += s_items[w];
        rbase += s_rows[w];
    }
    if (!has_bin) return;
    auto place = [&](bool valid, bool tgt, uint32_t dst, uint32_t row) {  // (held particles: the scatter)
        if (!valid) return;
        row_of[dst] = tgt ? row : ~0u;
        if (tgt) act_rows[row] = dst;
    };
    if (beg == end) {
        if (lane == 0) dir_n[bin] = 0;
        return;
    }
    if (over) {  // the reference order: the scatter's payload stays
        uint32_t seen_t = 0;
        for (uint32_t c0 = beg; c0 < end; c0 += 64) {
            const uint32_t slot = c0 + lane;
            const bool valid = slot < end;
            const uint32_t i = valid ? order[slot] : 0u;
            const bool tgt = is_target(valid, i);
            const uint64_t mt = __ballot(tgt);
            place(valid, tgt, slot, rbase + seen_t + (uint32_t)__popcll(mt & lt));
            seen_t += (uint32_t)__popcll(mt);
        }
        const uint32_t cnt = end - beg;
        for (uint32_t m = lane; m < nitems; m += 64) {
            const uint32_t left = cnt - m * tpi;
            worklist[wbase + m] = make_uint2(beg + m * tpi, left < tpi ? left : tpi);
        }
        if (lane == 0) dir_n[bin] = K + 1;
        return;
    }
    uint32_t seen[K], seen_t[K], rstart[K];
    {
        uint32_t r = rbase;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            seen[k] = 0;
            seen_t[k] = 0;
            rstart[k] = r;  // targets take rows in run order, slot order within a run
            r += gt[k];
        }
    }
    // one cell: the runs are the scatter's order and its payload stays; several cells are reordered
    // here (the held chunks from their sorted records, read in the first pass before any slot is
    // rewritten; later chunks from the step's input arrays)
    const bool rewrite = ng > 1;
    auto place_chunk = [&](bool valid, uint32_t i, const int c[3], const float4& p4, bool tgt) {
        const int gid = group_of(c);
        uint32_t dst = 0, row = 0;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint64_t m = __ballot(valid && gid == (int)k);
            const uint64_t mt = __ballot(tgt && gid == (int)k);
            if (gid == (int)k) {
                dst = start[k] + seen[k] + (uint32_t)__popcll(m & lt);
                row = rstart[k] + seen_t[k] + (uint32_t)__popcll(mt & lt);
            }
            seen[k] += (uint32_t)__popcll(m);
            seen_t[k] += (uint32_t)__popcll(mt);
        }
        if (valid && rewrite) write_sorted<D>(dst, i, b, n, p4, c, states, S, perm, inv, srec, scoord, sstate);
        place(valid, tgt, dst, row);
    };
#pragma unroll
    for (uint32_t k = 0; k < NH; ++k)
        if (beg + 64 * k < end) place_chunk(hv[k], hi[k], hc[k], hr[k], ht[k]);
    for (uint32_t c0 = beg + 64 * NH; c0 < end; c0 += 64) {
        bool valid;
        uint32_t i;
        float4 p4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        int c[3];
        if (rewrite) load(c0, valid, i, p4, c);
        else load_sorted(c0, valid, i, c);
        place_chunk(valid, i, c, p4, is_target(valid, i));
    }
    uint32_t off = 0;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        if (k < ng) {
            const uint32_t it = (gc[k] + tpi - 1) / tpi;
            for (uint32_t m = lane; m < it; m += 64) {
                const uint32_t left = gc[k] - m * tpi;
                worklist[wbase + off + m] = make_uint2(start[k] + m * tpi, left < tpi ? left : tpi);
            }
            off += it;
            if (lane == 0) dir_e[(uint64_t)bin * K + k] = make_int4(gx[k], gy[k], gz[k], (int)start[k]);
        }
    }
    if (lane == 0) dir_n[bin] = ng;
}

// The same split for sparse grids, one lane per bin: a bin of at most kThinMax particles is split
// by a single lane walking its slots in order (runs in order of first appearance, slot order
// within a run, the same work items, compact rows and directory entries as k_split); larger bins
// are listed for k_split. Used when bins outnumber a quarter of the particles, where a wave per
// bin would spend a whole wave's instructions on an empty or one-particle bin.
constexpr uint32_t kThinMax = kDirGroups;

constexpr uint32_t kThinThreads = 512;  // bins per k_split_thin block (one reservation each)

// Exclusive prefix of v over a kThinThreads block and the block's total.
__device__ __forceinline__ uint32_t block_prefix_thin(uint32_t v, uint32_t* ldsw, uint32_t* total) {
    constexpr uint32_t NW = kThinThreads / 64;
    const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const uint32_t x = wave_incl_add(v);
    if (lane == 63) ldsw[wid] = x;
    __syncthreads();
    uint32_t pre = 0, all = 0;
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w) {
        const uint32_t t = ldsw[w];
        if (w < wid) pre += t;
        all += t;
    }
    *total = all;
    return pre + x - v;
}

template <int D>
__global__ __launch_bounds__(kThinThreads) void k_split_thin(const float4* __restrict__ pos, const float* __restrict__ states,
                                                   uint32_t S, uint32_t n, uint32_t nbins, GridParams g,
                                                   const uint32_t* __restrict__ bo,
                                                   const uint32_t* __restrict__ order,
                                                   uint32_t* __restrict__ perm, uint32_t* __restrict__ inv,
                                                   float4* __restrict__ srec, int4* __restrict__ scoord,
                                                   float* __restrict__ sstate, uint32_t* __restrict__ dir_n,
                                                   int4* __restrict__ dir_e, uint2* __restrict__ worklist,
                                                   uint32_t* __restrict__ wl_count, uint32_t tpi, SplitTargets T,
                                                   uint32_t* __restrict__ act_rows, uint32_t* __restrict__ row_of,
                                                   uint32_t* __restrict__ bin_list) {
    constexpr uint32_t K = kDirGroups;
    __shared__ uint32_t lds_i[kThinThreads / 64], lds_r[kThinThreads / 64], lds_f[kThinThreads / 64];
    __shared__ uint32_t s_base[3];
    const uint32_t bin = blockIdx.x * blockDim.x + threadIdx.x;
    const bool has_bin = bin < nbins;
    const uint32_t beg = has_bin ? bo[bin] : 0u, end = has_bin ? bo[bin + 1] : 0u;
    const bool thin = has_bin && end - beg <= kThinMax;
    const bool fat = has_bin && !thin;
    const uint32_t b = has_bin ? bin / g.cells : 0u;
    auto is_target = [&](uint32_t i) -> bool {
        if (T.mask_mode == 0) return true;
        const uint32_t li = i - b * n;
        const float m = T.mask_mode == 1 ? hash_mask(li, b, n, T.update_prob, T.step_index, T.base_seed) : T.mask[i];
        return m != 0.0f;
    };
    // slot q's particle and cell from the scatter's sorted record
    auto load_sorted = [&](uint32_t q, uint32_t& i, int c[3]) {
        i = order[q];
        if constexpr (D == 2) {
            const float4 r = srec[q];
            c[0] = __float_as_int(r.z);
            c[1] = __float_as_int(r.w);
            c[2] = 0;
        } else {
            const int4 cc = scoord[q];
            c[0] = cc.x;
            c[1] = cc.y;
            c[2] = cc.z;
        }
    };
    int gx[K], gy[K], gz[K];
    uint32_t gc[K], gt[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        gx[k] = gy[k] = gz[k] = 0;
        gc[k] = gt[k] = 0;
    }
    uint32_t ng = 0;
    auto group_of = [&](const int c[3]) -> int {
        int gid = -1;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if (k < ng && c[0] == gx[k] && c[1] == gy[k] && c[2] == gz[k]) gid = (int)k;
        return gid;
    };
    // the bin's slots (at most kThinMax), loaded together and kept in registers for both passes
    uint32_t qi[kThinMax];
    int qc[kThinMax][3];
    bool qt[kThinMax];
    if (thin && beg < end) {
#pragma unroll
        for (uint32_t j = 0; j < kThinMax; ++j) load_sorted(beg + j < end ? beg + j : beg, qi[j], qc[j]);
#pragma unroll
        for (uint32_t j = 0; j < kThinMax; ++j) qt[j] = beg + j < end && is_target(qi[j]);
    }
    uint32_t nitems = 0, nrows = 0;
    if (thin) {  // pass 1: runs in order of first appearance, their particles and targets
#pragma unroll
        for (uint32_t j = 0; j < kThinMax; ++j) {
            if (beg + j >= end) break;
            const int* c = qc[j];
            int gid = group_of(c);
            if (gid < 0) {
                gid = (int)ng;
#pragma unroll
                for (uint32_t k = 0; k < K; ++k)
                    if (k == ng) {
                        gx[k] = c[0];
                        gy[k] = c[1];
                        gz[k] = c[2];
                    }
                ++ng;
            }
            const uint32_t t = qt[j] ? 1u : 0u;
#pragma unroll
            for (uint32_t k = 0; k < K; ++k)
                if ((int)k == gid) {
                    gc[k] += 1;
                    gt[k] += t;
                }
        }
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            nitems += (gc[k] + tpi - 1) / tpi;
            nrows += gt[k];
        }
    }
    // one reservation per block: work items, compact rows and listed bins
    uint32_t ti, tr, tf;
    const uint32_t pi_ = block_prefix_thin(nitems, lds_i, &ti);
    const uint32_t pr_ = block_prefix_thin(nrows, lds_r, &tr);
    const uint32_t pf_ = block_prefix_thin(fat ? 1u : 0u, lds_f, &tf);
    if (threadIdx.x == 0) {
        const unsigned long long add = (unsigned long long)ti | ((unsigned long long)tr << 32);
        const unsigned long long old = add ? atomicAdd(reinterpret_cast<unsigned long long*>(wl_count), add) : 0ull;
        s_base[0] = (uint32_t)old;
        s_base[1] = (uint32_t)(old >> 32);
        s_base[2] = tf ? atomicAdd(wl_count + kListedWord, tf) : 0u;
    }
    __syncthreads();
    if (fat) bin_list[s_base[2] + pf_] = bin;
    if (!thin) return;
    if (beg == end) {
        dir_n[bin] = 0;
        return;
    }
    // pass 2: slots in order; targets take rows in run order, slot order within a run
    const uint32_t wbase = s_base[0] + pi_, rbase = s_base[1] + pr_;
    uint32_t start[K], rstart[K], seen[K], seen_t[K];
    {
        uint32_t run = beg, r = rbase;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            start[k] = run;
            rstart[k] = r;
            run += gc[k];
            r += gt[k];
            seen[k] = seen_t[k] = 0;
        }
    }
    const bool rewrite = ng > 1;  // one cell: the scatter's payload is already in run order
#pragma unroll
    for (uint32_t j = 0; j < kThinMax; ++j) {
        if (beg + j >= end) break;
        const uint32_t i = qi[j];
        const int* c = qc[j];
        const int gid = group_of(c);
        const bool tgt = qt[j];
        uint32_t dst = 0, row = 0;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k)
            if ((int)k == gid) {
                dst = start[k] + seen[k];
                row = rstart[k] + seen_t[k];
                seen[k] += 1;
                seen_t[k] += tgt ? 1u : 0u;
            }
        // a reordered bin is rewritten from the step's input arrays (its cells are in registers)
        if (rewrite) write_sorted<D>(dst, i, b, n, pos[i], c, states, S, perm, inv, srec, scoord, sstate);
        row_of[dst] = tgt ? row : ~0u;
        if (tgt) act_rows[row] = dst;
    }
    uint32_t off = 0;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
        if (k < ng) {
            const uint32_t it = (gc[k] + tpi - 1) / tpi;
            for (uint32_t m = 0; m < it; ++m) {
                const uint32_t left = gc[k] - m * tpi;
                worklist[wbase + off + m] = make_uint2(start[k] + m * tpi, left < tpi ? left : tpi);
            }
            off += it;
            dir_e[(uint64_t)bin * K + k] = make_int4(gx[k], gy[k], gz[k], (int)start[k]);
        }
    }
    dir_n[bin] = ng;
}

// ------------------------------------------------ one block per system (small systems)
// The payload build of small systems in two launches instead of four (rank, offsets scan, payload
// scatter, split). Used when a system has at most kSysMaxCells bins (coordinate bins in Particle
// mode, cells in Grid mode) and at most kSysMaxRounds * 1024 particles (C1 and C5: 4,096 particles
// over 4,096 bins; more rounds per wave would spill registers).
// k_sys_rank, one 1024-thread block per system (wave w owns particles [w R 64, (w + 1) R 64)):
//   1. per particle its key and one LDS atomic on the key's counter (particles | update-mask
//      targets << 16), whose old value is the particle's place in its bin and, for a target, its
//      target index there - in whatever order the atomics land;
//   2. per key (thread t: keys 4t .. 4t + 3, read four at a time): one block scan of three sums:
//      the key's first slot (bin_offsets), its first work item (ceil(count / tpi) items of <= tpi
//      slots, as the split emits for a bin of one cell or an unsplit bin; sys_item[b][key]) and its
//      first compact row; the system's item and row totals go to sys_tot[b];
//   3. per particle: members[bin start + place] = particle (LDS);
//   4. per particle: its rank in the bin = the bin's members with a smaller index (the reference's
//      order within a bin; a bin of k particles costs each of them k LDS reads), its slot within the
//      system (keys[i]) and, for a target, its compact row = the bin's first row + its target index
//      (ranks[i] = row + 1, 0 for no row; bit 31 marks the bin's first particle). Rows only index
//      the targets, no result depends on their order.
// k_sys_scatter, one thread per particle, one wave per block (the waves spread over every CU): the
// systems' item and row bases (prefix of sys_tot, summed while the particle's position and state
// row are in flight), then the sorted record, state row and snapshot entries at the particle's
// slot, the work item starting
// there, its compact row (act_rows / row_of), the bin's directory entry from its first particle, and
// the step's output for a particle outside the update mask (hold_particle); block 0 writes the item
// and row totals and clears the update's item queues.
// A Particle-mode bin holds one cell unless two coordinates of the system's span share its residues
// on some axis; such bins are marked unsplit (dir_n = kDirGroups + 1: the neighbour passes walk the
// whole bin in the reference order and keep the cell's particles), which is exact for any bin. The
// coordinate-overflow flag goes to the sticky word flags[1] directly.
constexpr uint32_t kSysThreads = 1024;
constexpr uint32_t kSysWaves = kSysThreads / 64;

// cell_coords (hashgrid.rs:98-121) in 32-bit arithmetic: the same coordinates whenever they lie
// within +-2^30 (beyond that *overflow is set, as cell_coords sets it, and the coordinates only
// have to be some in-range value); a NaN coordinate is 0, as `f as isize` makes it. The key is the
// bin cell_of_coords gives (coordinate bins in Particle mode, the cell in Grid mode).
__device__ __forceinline__ void sys_cell(const float* p, const GridParams& g, int c[3], uint32_t* key,
                                         bool* overflow) {
    c[0] = c[1] = c[2] = 0;
    uint32_t h = 0, stride = 1;
    for (int a = 0; a < g.dim; ++a) {
        const float f = g.mode == 1 ? floorf(p[a] / g.eps) : floorf((p[a] + g.half[a]) / g.eps);
        const bool in = f >= -1073741824.0f && f <= 1073741824.0f;
        if (!in && f == f && g.mode == 1) *overflow = true;  // (Grid mode clamps or wraps below)
        int v = in ? (int)f : (f != f ? 0 : (f > 0.0f ? 1073741824 : -1073741824));
        const uint32_t m = g.size[a];
        if (g.mode == 1) {
            c[a] = v;
            const uint32_t w = (m & (m - 1)) == 0 ? (uint32_t)v & (m - 1) : (uint32_t)(((v % (int)m) + (int)m) % (int)m);
            h += w * stride;
        } else {
            if (g.boundary == 0) {  // rem_euclid of the full value (beyond 2^30 in 64-bit arithmetic)
                v = in ? ((v % (int)m) + (int)m) % (int)m : (int)rem_euclid_i64(f32_to_isize(f), (int64_t)m);
            } else {
                v = v < 0 ? 0 : (v > (int)m - 1 ? (int)m - 1 : v);
            }
            c[a] = v;
            h += (uint32_t)v * stride;
        }
        stride *= m;
    }
    *key = h;
}

constexpr uint32_t kSysMaxCells = 4096;
constexpr uint32_t kSysMaxRounds = 4;

__host__ __device__ inline uint32_t sys_row_stride(uint32_t C) { return (C + 3) & ~3u; }  // words per key row
// counters [cp] u32, first slots [cp + 4] u32, first rows [cp] u32, members [kSysMaxRounds * 1024] u16
inline uint32_t sys_lds_bytes(uint32_t C) { return 12u * sys_row_stride(C) + 16u + 2u * kSysMaxRounds * kSysThreads; }

template <int D, int R>
__global__ __launch_bounds__(kSysThreads) void k_sys_rank(const float4* __restrict__ pos, uint32_t n, GridParams g,
                                                          uint32_t tpi_log2, SplitTargets T,
                                                          uint32_t* __restrict__ bin_offsets,
                                                          uint32_t* __restrict__ dir_n, uint32_t* __restrict__ sys_item,
                                                          unsigned long long* __restrict__ sys_tot,
                                                          uint32_t* __restrict__ slot_of,
                                                          uint32_t* __restrict__ row_code, uint32_t batch,
                                                          uint32_t* __restrict__ flags) {
    extern __shared__ uint32_t sys_lds[];
    constexpr uint32_t K = kDirGroups;
    const uint32_t C = g.cells, cp = sys_row_stride(C);
    uint32_t* cnt = sys_lds;                     // per key: particles | update-mask targets << 16
    uint32_t* sstart = cnt + cp;                 // the key's first slot in the system
    uint32_t* srow = sstart + cp + 4;            // the key's first compact row in the system
    uint16_t* members = reinterpret_cast<uint16_t*>(srow + cp);  // the bins' particles, by bin
    __shared__ uint32_t red[3][kSysWaves];
    __shared__ int red_lo[3][kSysWaves], red_hi[3][kSysWaves];
    const uint32_t b = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const uint64_t sys = (uint64_t)b * n;

    for (uint32_t k = tid; k < cp / 4; k += kSysThreads) reinterpret_cast<uint4*>(cnt)[k] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    // ---- 1. keys, and one LDS atomic per particle on its key's counter: the old value is the
    // particle's place in its bin and, for a target, its target index there (in whatever order the
    // atomics land: the ranks below restore the reference's order, and rows only index targets)
    uint32_t key_r[R], place_r[R], tgt_bits = 0;
    int lo[3] = {INT32_MAX, INT32_MAX, INT32_MAX}, hi[3] = {INT32_MIN, INT32_MIN, INT32_MIN};
    bool ovf = false;
    float4 p_r[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = (w * R + r) * 64 + lane;
        p_r[r] = li < n ? pos[sys + li] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = (w * R + r) * 64 + lane;
        key_r[r] = 0;
        place_r[r] = 0;
        if (li < n) {
            const float p[4] = {p_r[r].x, p_r[r].y, p_r[r].z, p_r[r].w};
            int c[3];
            uint32_t key;
            sys_cell(p, g, c, &key, &ovf);
#pragma unroll
            for (int a = 0; a < D; ++a) {
                lo[a] = min(lo[a], c[a]);
                hi[a] = max(hi[a], c[a]);
            }
            const bool tgt = T.mask_mode == 0 ||
                             (T.mask_mode == 1 ? hash_mask(li, b, n, T.update_prob, T.step_index, T.base_seed)
                                               : T.mask[sys + li]) != 0.0f;
            const uint32_t old = atomicAdd(cnt + key, 1u | ((uint32_t)tgt << 16));
            key_r[r] = key;
            place_r[r] = old;
            if (tgt) tgt_bits |= 1u << r;
        }
    }
    // the system's coordinate span (Particle mode: do coordinate bins hold one cell each?)
#pragma unroll
    for (int a = 0; a < D; ++a) {
        const int l = wave_min_i32(lo[a]), h = wave_max_i32(hi[a]);
        if (lane == 0) {
            red_lo[a][w] = l;
            red_hi[a][w] = h;
        }
    }
    if (__ballot(ovf) != 0ull && lane == 0) atomicOr(flags + 1, 1u);
    __syncthreads();

    // ---- 2. per key (thread t: keys 4t .. 4t + 3): one block scan of three sums - the key's first
    // slot (bin_offsets), its first work item (ceil(count / tpi) items of <= tpi slots, as the split
    // emits for a bin of one cell or an unsplit bin; sys_item[b][key]) and its first compact row;
    // the system's item and row totals go to sys_tot[b]
    const uint32_t k0 = 4 * tid;
    uint32_t tot[4] = {0u, 0u, 0u, 0u}, msk[4] = {0u, 0u, 0u, 0u}, itm[4] = {0u, 0u, 0u, 0u};
    if (k0 < cp) {
        const uint4 v = reinterpret_cast<const uint4*>(cnt)[tid];
        const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            tot[q] = vv[q] & 0xffffu;
            msk[q] = vv[q] >> 16;
            itm[q] = (tot[q] + (1u << tpi_log2) - 1) >> tpi_log2;
        }
    }
    const uint32_t sa = tot[0] + tot[1] + tot[2] + tot[3];
    const uint32_t sb = itm[0] + itm[1] + itm[2] + itm[3];
    const uint32_t sm = msk[0] + msk[1] + msk[2] + msk[3];
    const uint32_t xa = wave_incl_add(sa), xb = wave_incl_add(sb), xm = wave_incl_add(sm);
    if (lane == 63) {
        red[0][w] = xa;
        red[1][w] = xb;
        red[2][w] = xm;
    }
    __syncthreads();
    // lane v < 16 holds wave v's sums: a 16-lane inclusive scan gives every wave its prefix
    uint32_t ea = 0, eb = 0, em = 0;
    if (lane < kSysWaves) {
        ea = red[0][lane];
        eb = red[1][lane];
        em = red[2][lane];
    }
    static_assert(kSysWaves == 16, "the waves' sums are scanned within lanes 0-15 (one DPP row)");
    ea = row_incl_add(ea);
    eb = row_incl_add(eb);
    em = row_incl_add(em);
    // earlier waves' sums (w is wave-uniform)
    const uint32_t pa = w ? (uint32_t)__builtin_amdgcn_readlane((int)ea, (int)w - 1) : 0u;
    const uint32_t pb = w ? (uint32_t)__builtin_amdgcn_readlane((int)eb, (int)w - 1) : 0u;
    const uint32_t pm = w ? (uint32_t)__builtin_amdgcn_readlane((int)em, (int)w - 1) : 0u;
    const uint32_t tb = (uint32_t)__builtin_amdgcn_readlane((int)eb, (int)kSysWaves - 1);
    const uint32_t tm = (uint32_t)__builtin_amdgcn_readlane((int)em, (int)kSysWaves - 1);
    // the system's coordinate span per axis: a bin may hold two cells only if two coordinates of the
    // span share its residue on some axis (see k_bin_scan); no axis wider than the grid, no alias
    int span_lo_a[3] = {0, 0, 0}, span_hi_a[3] = {0, 0, 0};
    bool wide = false;
    if (g.mode == 1) {
#pragma unroll
        for (int a = 0; a < D; ++a) {
            span_lo_a[a] = wave_min_i32(lane < kSysWaves ? red_lo[a][lane] : INT32_MAX);
            span_hi_a[a] = wave_max_i32(lane < kSysWaves ? red_hi[a][lane] : INT32_MIN);
            if (span_hi_a[a] >= span_lo_a[a] && (int64_t)span_hi_a[a] - span_lo_a[a] >= (int64_t)g.size[a]) wide = true;
        }
    }
    auto may_alias = [&](uint32_t k) {
        bool al = false;
        uint32_t rest = k;
#pragma unroll
        for (int a = 0; a < D; ++a) {
            const int64_t m = (int64_t)g.size[a];
            const int64_t r = (int64_t)(rest % g.size[a]);
            rest /= g.size[a];
            const int64_t l = span_lo_a[a], h = span_hi_a[a];
            if (h >= l && h - l >= m && l + rem_euclid_i64(r - l, m) + m <= h) al = true;
        }
        return al;
    };
    if (tid == 0) {
        sys_tot[b] = (unsigned long long)tb | ((unsigned long long)tm << 32);
        if (b == batch - 1) bin_offsets[(uint64_t)batch * C] = batch * n;
    }
    if (k0 < C) {
        uint32_t st = pa + xa - sa, it = pb + xb - sb, rw = pm + xm - sm;
        uint32_t sv[4], rv[4], ov[4], iv[4], dv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t k = k0 + q;
            sv[q] = st;
            rv[q] = rw;
            ov[q] = b * n + st;
            iv[q] = it;
            dv[q] = k < C && g.mode == 1 && tot[q] ? (wide && may_alias(k) ? K + 1 : 1u) : 0u;
            st += tot[q];
            it += itm[q];
            rw += msk[q];
        }
        const uint64_t at = (uint64_t)b * C + k0;
        if (k0 + 3 < C && (C & 3u) == 0) {  // one 16-byte store per array (aligned when C % 4 == 0)
            *reinterpret_cast<uint4*>(bin_offsets + at) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
            *reinterpret_cast<uint4*>(sys_item + at) = make_uint4(iv[0], iv[1], iv[2], iv[3]);
            if (g.mode == 1) *reinterpret_cast<uint4*>(dir_n + at) = make_uint4(dv[0], dv[1], dv[2], dv[3]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (k0 + q < C) {
                    bin_offsets[at + q] = ov[q];
                    sys_item[at + q] = iv[q];
                    if (g.mode == 1) dir_n[at + q] = dv[q];
                }
            }
        }
        reinterpret_cast<uint4*>(sstart)[tid] = make_uint4(sv[0], sv[1], sv[2], sv[3]);
        reinterpret_cast<uint4*>(srow)[tid] = make_uint4(rv[0], rv[1], rv[2], rv[3]);
    }
    __syncthreads();

    // ---- 3. each particle at its bin's start + its place, then 4. its rank in the bin = the bin's
    // members with a smaller index (the reference's order), hence its slot; a target's row is the
    // bin's first row + its target index; bit 31 marks the bin's first particle
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = (w * R + r) * 64 + lane;
        if (li < n) members[sstart[key_r[r]] + (place_r[r] & 0xffffu)] = (uint16_t)li;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t li = (w * R + r) * 64 + lane;
        if (li >= n) continue;
        const uint32_t key = key_r[r];
        const uint32_t beg = sstart[key], end = beg + (cnt[key] & 0xffffu);
        uint32_t rank = 0;
        for (uint32_t j = beg; j < end; ++j) rank += (uint32_t)members[j] < li ? 1u : 0u;
        uint32_t code = rank == 0 ? 0x80000000u : 0u;
        if ((tgt_bits >> r) & 1u) code |= srow[key] + (place_r[r] >> 16) + 1u;
        slot_of[sys + li] = beg + rank;
        row_code[sys + li] = code;
    }
}

template <int D, int NQ>
__global__ __launch_bounds__(64) void k_sys_scatter(const float4* __restrict__ pos, const float* __restrict__ states,
                                                    uint32_t S, uint32_t n, uint32_t batch, GridParams g,
                                                    uint32_t tpi_log2, SplitTargets T,
                                                    const uint32_t* __restrict__ bin_offsets,
                                                    const uint32_t* __restrict__ sys_item,
                                                    const unsigned long long* __restrict__ sys_tot,
                                                    const uint32_t* __restrict__ slot_of,
                                                    const uint32_t* __restrict__ row_code,
                                                    uint32_t* __restrict__ perm, uint32_t* __restrict__ inv,
                                                    float4* __restrict__ srec, int4* __restrict__ scoord,
                                                    float* __restrict__ sstate, int4* __restrict__ dir_e,
                                                    uint2* __restrict__ worklist, uint32_t* __restrict__ wl_count,
                                                    uint32_t* __restrict__ act_rows, uint32_t* __restrict__ row_of) {
    const uint32_t lane = threadIdx.x;  // one wave per block
    const uint64_t total = (uint64_t)batch * n;
    const uint64_t first = (uint64_t)blockIdx.x * 64;  // < total
    const uint32_t b_lo = (uint32_t)(first / n);       // the block's first system
    const uint64_t i = first + lane;
    const bool live = i < total;
    // the particle's inputs (the state row when NQ > 0: NQ float4s, 16-byte aligned rows) are
    // independent of the systems' bases: in flight while those are summed
    const uint64_t ii = live ? i : first;
    const float4 p4 = pos[ii];
    const uint32_t local = slot_of[ii];
    const uint32_t code = row_code[ii];
    float4 row[NQ > 0 ? NQ : 1];
    if constexpr (NQ > 0) {
        const float4* src = reinterpret_cast<const float4*>(states + ii * S);
#pragma unroll
        for (int q = 0; q < NQ; ++q) row[q] = src[q];
    }
    // item and row bases of the block's systems: prefix sums of the systems' totals (items in the
    // low word, rows in the high word: no carries, both stay below 2^32); block 0 also sums them all
    const uint32_t upto = blockIdx.x == 0 ? batch : b_lo;
    unsigned long long acc = 0;
    for (uint32_t k = lane; k < upto; k += 64) acc += sys_tot[k];
    const uint32_t all_items = wave_sum_u32((uint32_t)acc), all_rows = wave_sum_u32((uint32_t)(acc >> 32));
    if (blockIdx.x == 0) {  // the lists' counts; the update's item queues start at zero
        if (lane == 0) {
            wl_count[0] = all_items;
            wl_count[1] = all_rows;
        }
        for (uint32_t k = 2 + lane; k < kWlWords; k += 64) wl_count[k] = 0u;
    }
    if (!live) return;
    const uint32_t b = (uint32_t)(i / n);
    unsigned long long base = blockIdx.x == 0 ? 0ull : ((unsigned long long)all_rows << 32) | all_items;
    for (uint32_t bb = b_lo; bb < b; ++bb) base += sys_tot[bb];  // a block spanning several systems
    const uint32_t ibase = (uint32_t)base, rbase = (uint32_t)(base >> 32);
    const float p[4] = {p4.x, p4.y, p4.z, p4.w};
    int c[3];
    uint32_t key;
    bool o = false;
    sys_cell(p, g, c, &key, &o);  // (an overflow was flagged by the rank kernel)
    const uint64_t bin = (uint64_t)b * g.cells + key;
    const uint32_t beg = bin_offsets[bin], nxt = bin_offsets[bin + 1], item0 = sys_item[bin];
    // used here, so the bin's loads are issued together (read-only loads are otherwise moved down to
    // their uses, after the stores)
    asm volatile("" ::"v"(beg), "v"(nxt), "v"(item0));
    if constexpr (NQ > 0) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) asm volatile("" ::"v"(row[q].x), "v"(row[q].y), "v"(row[q].z), "v"(row[q].w));
    }
    const uint32_t slot = b * n + local;
    write_sorted<D>(slot, (uint32_t)i, b, n, p4, c, NQ > 0 ? nullptr : states, S, perm, inv, srec, scoord, sstate);
    if constexpr (NQ > 0) {
        float4* o4 = reinterpret_cast<float4*>(sstate + (uint64_t)slot * (4 * NQ));
#pragma unroll
        for (int q = 0; q < NQ; ++q) o4[q] = row[q];
    }
    const uint32_t row1 = code & 0x7fffffffu;
    if (row1) {
        const uint32_t crow = rbase + row1 - 1u;
        act_rows[crow] = slot;
        row_of[slot] = crow;
    } else {
        row_of[slot] = ~0u;
        if (T.mask_mode != 0) {
            bool held = false;
            if constexpr (NQ > 0) {
                if (T.pos == pos && T.states == states) {  // the step's input rows, already loaded
                    hold_loaded<NQ>(i, p4, row, g, T.out_pos, T.out_states);
                    held = true;
                }
            }
            if (!held) hold_particle(i, S, g, T.pos, T.states, T.out_pos, T.out_states);
        }
    }
    const uint32_t r_bin = slot - beg;
    const uint32_t tpi = 1u << tpi_log2;
    if ((r_bin & (tpi - 1)) == 0) {
        const uint32_t left = nxt - beg - r_bin;
        worklist[ibase + item0 + (r_bin >> tpi_log2)] = make_uint2(slot, left < tpi ? left : tpi);
    }
    if (g.mode == 1 && (code >> 31)) dir_e[bin * kDirGroups] = make_int4(c[0], c[1], c[2], (int)slot);
}

// The small-system scatter for the state width: rows preloaded when they are whole float4s.
template <int D>
static auto sys_scatter_for(const float* states, uint32_t S) -> decltype(&k_sys_scatter<D, 0>) {
    if (!states || S != state_stride_for(S)) return k_sys_scatter<D, 0>;
    switch (S / 4) {
        case 1: return k_sys_scatter<D, 1>;
        case 2: return k_sys_scatter<D, 2>;
        case 4: return k_sys_scatter<D, 4>;
        case 6: return k_sys_scatter<D, 6>;
        default: return k_sys_scatter<D, 8>;
    }
}

template <int D, int R>
static hipError_t launch_sys_r(const GridParams& g, const HashgridPlan& plan, const float4* pos, const float* states,
                               uint32_t S, uint32_t batch, uint32_t n, Workspace& ws, const SplitTargets& tg,
                               hipStream_t stream, Profiler* prof) {
    const uint32_t lds = sys_lds_bytes(plan.cells);
    if (lds > 32768) {
        static LdsLimitFlags limit;
        const hipError_t e = raise_lds_limit((const void*)k_sys_rank<D, R>, limit);
        if (e != hipSuccess) return e;
    }
    // per particle: slot (keys) and row code (ranks); per bin: first item (totals); per system: totals
    hipError_t e = launch_timed(prof, NPA_KERNEL_HASH_RANK, k_sys_rank<D, R>, dim3(batch), dim3(kSysThreads), lds,
                                stream, pos, n, g, (uint32_t)__builtin_ctz(plan.tpi), tg,
                                ws.bin_offsets.as<uint32_t>(),
                                ws.dir_n.as<uint32_t>(), ws.totals.as<uint32_t>(),
                                ws.scan_status.as<unsigned long long>(), ws.keys.as<uint32_t>(),
                                ws.ranks.as<uint32_t>(), batch, ws.flags.as<uint32_t>());
    if (e != hipSuccess) return e;
    const uint64_t total = (uint64_t)batch * n;
    return launch_timed(prof, NPA_KERNEL_SCATTER, sys_scatter_for<D>(states, S), dim3((uint32_t)((total + 63) / 64)), dim3(64),
                        0, stream, pos, states, S, n, batch, g, (uint32_t)__builtin_ctz(plan.tpi), tg,
                        ws.bin_offsets.as<uint32_t>(),
                        ws.totals.as<uint32_t>(), ws.scan_status.as<unsigned long long>(), ws.keys.as<uint32_t>(),
                        ws.ranks.as<uint32_t>(), ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(),
                        ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(), ws.dir_e.as<int4>(),
                        ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), ws.act_rows.as<uint32_t>(),
                        ws.row_of.as<uint32_t>());
}

// ------------------------------------------------ binned build (one system)
// The payload build of one system whose bins are cells (Grid mode) or coordinate bins (Particle
// mode) in four launches, with no per-tile tables:
//   k_bin_count   per particle: its bin, and one 64-bit atomic on the bin's counter (particles in
//                 the low half, update-mask targets in the high half) whose old value gives the
//                 particle a place within its bin and, for a target, a target index within it -
//                 both in whatever order the atomics land; the cell coordinate span (six atomic
//                 maxima); block 0 clears the work-list counters, every block its share of the
//                 offsets scan's status words;
//   k_bin_scan    per bin (2,048 per 512-thread block, four per thread): the exclusive prefixes
//                 of the counts (bin_offsets), of the work items (ceil(count / tpi) items of <= tpi
//                 slots, as the split emits for a bin of one cell or an unsplit bin) and of the
//                 targets (the bin's first compact row), with decoupled look-back over
//                 ticket-ordered blocks; the directory sizes; it resets the counters and the span
//                 for the next build;
//   k_bin_place   per particle: members[bin start + place] = particle;
//   k_bin_scatter per particle (place and scatter run one wave per block, so that the few waves of a
//                 small system spread over every CU; the position and state row are loaded before
//                 the slot is known): its rank in the bin = the bin's members with a smaller index (the
//                 reference's order within a bin), hence its slot; then what k_scatter_payload
//                 writes there, its compact row (the bin's first row + its target index: rows only
//                 index the targets, no result depends on their order), the work item that starts
//                 at its slot and the bin's directory entry.
// A bin of k particles costs each of its particles k member reads in k_bin_scatter: a crowded
// bin makes that pass slower (O(k) per particle) but never wrong.
// Span words (after the counters): [a] = max of ~u(c_a) (the minimum), [3 + a] = max of u(c_a) (the
// maximum), u(v) = v ^ 0x80000000 (order-preserving), so that zero is the identity of both.
__device__ __forceinline__ uint32_t span_key(int v) { return (uint32_t)v ^ 0x80000000u; }
__device__ __forceinline__ int span_lo(uint32_t w) { return (int)(~w ^ 0x80000000u); }
__device__ __forceinline__ int span_hi(uint32_t w) { return (int)(w ^ 0x80000000u); }

template <int D>
__global__ __launch_bounds__(256) void k_bin_count(const float4* __restrict__ pos, uint32_t n, GridParams g,
                                                   SplitTargets T, unsigned long long* __restrict__ count,
                                                   uint32_t* __restrict__ span, uint32_t* __restrict__ keys,
                                                   uint32_t* __restrict__ place, uint32_t* __restrict__ urow,
                                                   uint32_t* __restrict__ wl_count,
                                                   unsigned long long* __restrict__ status, uint32_t nstatus,
                                                   uint32_t* __restrict__ flags) {
    __shared__ uint32_t red[6][4];
    const uint32_t i = blockIdx.x * 256 + threadIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (blockIdx.x == 0)
        for (uint32_t k = threadIdx.x; k < kWlWords; k += 256) wl_count[k] = 0u;
    for (uint32_t k = i; k < nstatus; k += gridDim.x * 256) status[k] = 0ull;
    uint32_t lo[3] = {0u, 0u, 0u}, hi[3] = {0u, 0u, 0u};
    bool ovf = false;
    if (i < n) {
        const float4 p4 = pos[i];
        const float p[4] = {p4.x, p4.y, p4.z, p4.w};
        int64_t c[3];
        cell_coords(p, g, c, &ovf);
        const uint32_t key = cell_of_coords(c, g);
#pragma unroll
        for (int a = 0; a < D; ++a) {
            const int v = (int)(c[a] < INT32_MIN ? INT32_MIN : (c[a] > INT32_MAX ? INT32_MAX : c[a]));
            lo[a] = ~span_key(v);
            hi[a] = span_key(v);
        }
        const bool tgt = T.mask_mode == 0 ||
                         (T.mask_mode == 1 ? hash_mask(i, 0, n, T.update_prob, T.step_index, T.base_seed) : T.mask[i]) != 0.0f;
        const unsigned long long old = atomicAdd(count + key, 1ull | ((unsigned long long)tgt << 32));
        keys[i] = key;
        place[i] = (uint32_t)old;
        urow[i] = tgt ? (uint32_t)(old >> 32) : ~0u;
    }
    if (__ballot(ovf) != 0ull && lane == 0) atomicOr(flags + 1, 1u);
#pragma unroll
    for (int a = 0; a < D; ++a) {
        lo[a] = wave_max_u32(lo[a]);
        hi[a] = wave_max_u32(hi[a]);
    }
    if (lane == 0)
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            red[a][w] = lo[a];
            red[3 + a][w] = hi[a];
        }
    __syncthreads();
    if (threadIdx.x < 6) {
        const uint32_t m = max(max(red[threadIdx.x][0], red[threadIdx.x][1]), max(red[threadIdx.x][2], red[threadIdx.x][3]));
        if (m) atomicMax(span + threadIdx.x, m);
    }
}

template <int W>
__global__ __launch_bounds__(64 * W) void k_bin_scan(unsigned long long* __restrict__ count, uint32_t* __restrict__ span,
                                                   uint32_t C, uint32_t tpi_log2, GridParams g,
                                                   unsigned long long* __restrict__ status,
                                                   uint32_t* __restrict__ bin_offsets, uint32_t* __restrict__ item_base,
                                                   uint32_t* __restrict__ row_base, uint32_t* __restrict__ dir_n,
                                                   uint32_t* __restrict__ wl_count) {
    // 256 W keys per block (W waves), four per thread (thread t: keys 4t .. 4t + 3 of the block's range)
    static_assert(W >= 1 && W <= 16, "the waves' sums are scanned within lanes 0 .. W - 1 (one DPP row)");
    __shared__ uint32_t red[3][W];
    __shared__ int s_span[6];
    __shared__ uint32_t s_pa, s_pb, s_pm, s_ticket;
    const uint32_t nb = gridDim.x, tid = threadIdx.x;
    if (tid == 0) s_ticket = (uint32_t)atomicAdd(status + 2ull * nb, 1ull);
    if (tid < 6) s_span[tid] = tid < 3 ? span_lo(span[tid]) : span_hi(span[tid]);
    __syncthreads();
    const uint32_t bx = s_ticket;
    const uint32_t k0 = (bx * (64 * W) + tid) * 4;
    const uint32_t lane = tid & 63, w = tid >> 6;
    uint32_t run[4], msk[4], itm[4];
    unsigned long long cv[4];
    if (k0 + 3 < C) {  // the thread's four counters in two 16-byte loads
        const ulonglong2 a = reinterpret_cast<const ulonglong2*>(count + k0)[0];
        const ulonglong2 c2 = reinterpret_cast<const ulonglong2*>(count + k0)[1];
        cv[0] = a.x;
        cv[1] = a.y;
        cv[2] = c2.x;
        cv[3] = c2.y;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) cv[q] = k0 + q < C ? count[k0 + q] : 0ull;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned long long v = cv[q];
        if (v) count[k0 + q] = 0ull;  // ready for the next build
        run[q] = (uint32_t)v;
        msk[q] = (uint32_t)(v >> 32);
        itm[q] = (run[q] + (1u << tpi_log2) - 1) >> tpi_log2;
    }
    const uint32_t sa = run[0] + run[1] + run[2] + run[3];
    const uint32_t sb = itm[0] + itm[1] + itm[2] + itm[3];
    const uint32_t sm = msk[0] + msk[1] + msk[2] + msk[3];
    const uint32_t xa = wave_incl_add(sa), xb = wave_incl_add(sb), xm = wave_incl_add(sm);
    if (lane == 63) {
        red[0][w] = xa;
        red[1][w] = xb;
        red[2][w] = xm;
    }
    __syncthreads();
    // lane v < W holds wave v's sums: an inclusive scan over the row gives every wave its prefix
    uint32_t ea = 0, eb = 0, em = 0;
    if (lane < W) {
        ea = red[0][lane];
        eb = red[1][lane];
        em = red[2][lane];
    }
    ea = row_incl_add(ea);
    eb = row_incl_add(eb);
    em = row_incl_add(em);
    // earlier waves' sums (w is wave-uniform)
    const uint32_t pa = w ? (uint32_t)__builtin_amdgcn_readlane((int)ea, (int)w - 1) : 0u;
    const uint32_t pb = w ? (uint32_t)__builtin_amdgcn_readlane((int)eb, (int)w - 1) : 0u;
    const uint32_t pm = w ? (uint32_t)__builtin_amdgcn_readlane((int)em, (int)w - 1) : 0u;
    const uint32_t ta = (uint32_t)__builtin_amdgcn_readlane((int)ea, W - 1);
    const uint32_t tb = (uint32_t)__builtin_amdgcn_readlane((int)eb, W - 1);
    const uint32_t tm = (uint32_t)__builtin_amdgcn_readlane((int)em, W - 1);
    // A coordinate bin (residues r_a = c_a mod size_a) can hold two cells only if on some axis two
    // coordinates of the span [lo, hi] share its residue: first = lo + ((r - lo) mod size) and
    // first + size <= hi. Such bins are marked unsplit (walked in the reference order with the cell
    // filter, exact for any bin); every other occupied bin holds one cell.
    bool wide = false;
#pragma unroll
    for (int a = 0; a < 3; ++a)
        if (a < g.dim && s_span[3 + a] >= s_span[a] && (int64_t)s_span[3 + a] - s_span[a] >= (int64_t)g.size[a]) wide = true;
    auto alias_of = [&](uint32_t k) {
        bool al = false;
        uint32_t rest = k;
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            if (a < g.dim) {
                const int64_t m = (int64_t)g.size[a];
                const int64_t r = (int64_t)(rest % g.size[a]);
                rest /= g.size[a];
                const int64_t l = s_span[a], h = s_span[3 + a];
                if (h >= l && h - l >= m && l + rem_euclid_i64(r - l, m) + m <= h) al = true;
            }
        }
        return al;
    };
    if (tid == 0) {
        __hip_atomic_store(status + bx, (1ull << 63) | ta, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(status + nb + bx, (1ull << 63) | tb | ((unsigned long long)tm << 31), __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    if (w == 0) {  // the earlier blocks' totals, 64 at a time (they took smaller tickets: running)
        uint32_t acc_a = 0, acc_b = 0, acc_m = 0;
        for (uint32_t base = 0; base < bx; base += 64) {
            const uint32_t j = base + lane;
            if (j < bx) {
                unsigned long long qa, qb;
                do {
                    qa = __hip_atomic_load(status + j, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                } while (!(qa >> 63));
                do {
                    qb = __hip_atomic_load(status + nb + j, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
                } while (!(qb >> 63));
                acc_a += (uint32_t)qa;
                acc_b += (uint32_t)(qb & 0x7fffffffull);
                acc_m += (uint32_t)((qb >> 31) & 0x7fffffffull);
            }
        }
        acc_a = wave_sum_u32(acc_a);
        acc_b = wave_sum_u32(acc_b);
        acc_m = wave_sum_u32(acc_m);
        if (lane == 0) {
            s_pa = acc_a;
            s_pb = acc_b;
            s_pm = acc_m;
        }
    }
    __syncthreads();
    uint32_t st = s_pa + pa + xa - sa, it = s_pb + pb + xb - sb, rw = s_pm + pm + xm - sm;
    uint32_t ov[4], iv[4], rv[4], dv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t k = k0 + q;
        ov[q] = st;
        iv[q] = it;
        rv[q] = rw;
        dv[q] = k < C && g.mode == 1 && run[q] ? (wide && alias_of(k) ? kDirGroups + 1 : 1u) : 0u;
        st += run[q];
        it += itm[q];
        rw += msk[q];
    }
    if (k0 + 3 < C) {  // the thread's four keys with one 16-byte store per array
        *reinterpret_cast<uint4*>(bin_offsets + k0) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
        *reinterpret_cast<uint4*>(item_base + k0) = make_uint4(iv[0], iv[1], iv[2], iv[3]);
        *reinterpret_cast<uint4*>(row_base + k0) = make_uint4(rv[0], rv[1], rv[2], rv[3]);
        if (g.mode == 1) *reinterpret_cast<uint4*>(dir_n + k0) = make_uint4(dv[0], dv[1], dv[2], dv[3]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t k = k0 + q;
            if (k < C) {
                bin_offsets[k] = ov[q];
                item_base[k] = iv[q];
                row_base[k] = rv[q];
                if (g.mode == 1) dir_n[k] = dv[q];
            }
        }
    }
    // the last ticket: every other block has read the span and published (its look-back saw them all)
    if (bx == nb - 1 && tid == 0) {
        bin_offsets[C] = s_pa + ta;
        wl_count[0] = s_pb + tb;
        wl_count[1] = s_pm + tm;
    }
    if (bx == nb - 1 && tid < 6) span[tid] = 0u;
}

__global__ __launch_bounds__(64) void k_bin_place(uint32_t n, const uint32_t* __restrict__ keys,
                                                   const uint32_t* __restrict__ place,
                                                   const uint32_t* __restrict__ bin_offsets,
                                                   uint32_t* __restrict__ members) {
    const uint32_t i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) members[bin_offsets[keys[i]] + place[i]] = i;
}

template <int D, int NQ>
__global__ __launch_bounds__(64) void k_bin_scatter(uint32_t n, const uint32_t* __restrict__ keys,
                                                     const uint32_t* __restrict__ urow,
                                                     const uint32_t* __restrict__ bin_offsets,
                                                     const uint32_t* __restrict__ members,
                                                     const uint32_t* __restrict__ item_base,
                                                     const uint32_t* __restrict__ row_base, uint32_t tpi_log2,
                                                     const float4* __restrict__ pos, const float* __restrict__ states,
                                                     uint32_t S, GridParams g, uint32_t* __restrict__ perm,
                                                     uint32_t* __restrict__ inv, float4* __restrict__ srec,
                                                     int4* __restrict__ scoord, float* __restrict__ sstate,
                                                     SplitTargets T, uint2* __restrict__ worklist,
                                                     uint32_t* __restrict__ act_rows, uint32_t* __restrict__ row_of,
                                                     int4* __restrict__ dir_e) {
    const uint32_t i = blockIdx.x * 64 + threadIdx.x;
    if (i >= n) return;
    // the position and state row (NQ > 0: NQ float4s, 16-byte aligned rows) are independent of the
    // slot: in flight while the rank is counted
    const float4 p4 = pos[i];
    float4 row[NQ > 0 ? NQ : 1];
    if constexpr (NQ > 0) {
        const float4* src = reinterpret_cast<const float4*>(states + (uint64_t)i * S);
#pragma unroll
        for (int q = 0; q < NQ; ++q) row[q] = src[q];
    }
    const uint32_t key = keys[i], ur = urow[i];
    const uint32_t beg = bin_offsets[key], end = bin_offsets[key + 1];
    const uint32_t rb = row_base[key], ib = item_base[key];
    // used here, so these loads are issued together (read-only loads are otherwise moved down to
    // their uses, after the member walk and the cell coordinates)
    asm volatile("" ::"v"(rb), "v"(ib));
    if constexpr (NQ > 0) {
        asm volatile("" ::"v"(p4.x), "v"(p4.y), "v"(p4.z), "v"(p4.w));
#pragma unroll
        for (int q = 0; q < NQ; ++q) asm volatile("" ::"v"(row[q].x), "v"(row[q].y), "v"(row[q].z), "v"(row[q].w));
    }
    uint32_t r = 0, j = beg;
    for (; j + 4 <= end; j += 4) {
        const uint32_t m0 = members[j], m1 = members[j + 1], m2 = members[j + 2], m3 = members[j + 3];
        r += (uint32_t)(m0 < i) + (uint32_t)(m1 < i) + (uint32_t)(m2 < i) + (uint32_t)(m3 < i);
    }
    for (; j < end; ++j) r += (uint32_t)(members[j] < i);
    const uint32_t dst = beg + r;
    const float p[4] = {p4.x, p4.y, p4.z, p4.w};
    int64_t c64[3];
    bool ovf = false;
    cell_coords(p, g, c64, &ovf);
    const int c[3] = {(int)c64[0], (int)c64[1], (int)c64[2]};
    write_sorted<D>(dst, i, 0, n, p4, c, NQ > 0 ? nullptr : states, S, perm, inv, srec, scoord, sstate);
    if constexpr (NQ > 0) {
        float4* o4 = reinterpret_cast<float4*>(sstate + (uint64_t)dst * (4 * NQ));
#pragma unroll
        for (int q = 0; q < NQ; ++q) o4[q] = row[q];
    }
    const bool tgt = ur != ~0u;
    if (tgt) {
        const uint32_t crow = rb + ur;
        act_rows[crow] = dst;
        row_of[dst] = crow;
    } else {
        row_of[dst] = ~0u;
        bool held = false;
        if constexpr (NQ > 0) {
            if (T.pos == pos && T.states == states) {  // the step's input rows, already loaded
                hold_loaded<NQ>(i, p4, row, g, T.out_pos, T.out_states);
                held = true;
            }
        }
        if (!held) hold_particle(i, S, g, T.pos, T.states, T.out_pos, T.out_states);
    }
    const uint32_t tpi = 1u << tpi_log2;
    if ((r & (tpi - 1)) == 0) {
        const uint32_t left = end - dst;
        worklist[ib + (r >> tpi_log2)] = make_uint2(dst, left < tpi ? left : tpi);
    }
    if (g.mode == 1 && r == 0) dir_e[(uint64_t)key * kDirGroups] = make_int4(c[0], c[1], c[2], (int)dst);
}

// The binned scatter for the state width: rows preloaded when they are whole float4s.
template <int D>
static auto bin_scatter_for(const float* states, uint32_t S) -> decltype(&k_bin_scatter<D, 0>) {
    if (!states || S != state_stride_for(S)) return k_bin_scatter<D, 0>;
    switch (S / 4) {
        case 1: return k_bin_scatter<D, 1>;
        case 2: return k_bin_scatter<D, 2>;
        case 4: return k_bin_scatter<D, 4>;
        case 6: return k_bin_scatter<D, 6>;
        default: return k_bin_scatter<D, 8>;
    }
}

// The binned build applies to a payload build of one system whose bins are cells or coordinate bins,
// with at most 8 particles per bin on average. (Measured against the folded build on the 2D C2 grid:
// faster at 2 and 4 particles per bin, equal at 8, 3 % slower at 16, where its count atomics queue
// 16 deep on each counter and the folded build's tile tables are small for the particles they
// rank; on C4's sparse 3D grid, 0.5 per bin, 14.5 us faster per step.)
static bool bin_build_applies(const HashgridPlan& plan, const GridParams& g, uint32_t batch, uint32_t n) {
    return batch == 1 && n > 0 && plan.cells > 0 && (uint64_t)n <= 8ull * plan.cells &&
           (plan.tpi & (plan.tpi - 1)) == 0 && plan.tpi <= 64 && (g.mode != 1 || g.spatial);
}

__global__ __launch_bounds__(256) void k_clear_u64(unsigned long long* __restrict__ a, uint32_t n) {
    for (uint32_t k = blockIdx.x * 256 + threadIdx.x; k < n; k += gridDim.x * 256) a[k] = 0ull;
}

static hipError_t launch_bins(const HashgridPlan& plan, const GridParams& g, const float4* pos, const float* states,
                              uint32_t S, uint32_t n, Workspace& ws, const SplitTargets& tg, hipStream_t stream,
                              Profiler* prof) {
    constexpr int kScanWaves = 8;  // k_bin_scan: 256 keys per wave (C4: 16 blocks; 16 waves were 0.4 us slower)
    const uint32_t C = plan.cells, blocks = (n + 255) / 256, kblocks = (C + 256 * kScanWaves - 1) / (256 * kScanWaves);
    const uint32_t tpi_log2 = (uint32_t)__builtin_ctz(plan.tpi);
    unsigned long long* count = ws.bin_count.as<unsigned long long>();
    uint32_t* span = reinterpret_cast<uint32_t*>(count + C);
    hipError_t e;
    if (!ws.bin_count.owned) {  // a carved workspace: its counters hold whatever the memory held
        const uint32_t words = C + 4;  // the counters and the span words, as 64-bit words
        hipLaunchKernelGGL(k_clear_u64, dim3(std::min<uint32_t>((words + 255) / 256, 1024)), dim3(256), 0, stream,
                           count, words);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    e = launch_timed(prof, NPA_KERNEL_HASH_RANK, g.dim == 2 ? k_bin_count<2> : k_bin_count<3>, dim3(blocks), dim3(256), 0,
                     stream, pos, n, g, tg, count, span, ws.keys.as<uint32_t>(), ws.ranks.as<uint32_t>(),
                     ws.bin_urow.as<uint32_t>(), ws.wl_count.as<uint32_t>(), ws.scan_status.as<unsigned long long>(),
                     2 * kblocks + 1, ws.flags.as<uint32_t>());
    if (e != hipSuccess) return e;
    e = launch_timed(prof, NPA_KERNEL_TABLE_SCAN, k_bin_scan<kScanWaves>, dim3(kblocks), dim3(64 * kScanWaves), 0, stream, count, span, C,
                     tpi_log2, g, ws.scan_status.as<unsigned long long>(), ws.bin_offsets.as<uint32_t>(),
                     ws.totals.as<uint32_t>(), ws.bin_list.as<uint32_t>(), ws.dir_n.as<uint32_t>(),
                     ws.wl_count.as<uint32_t>());
    if (e != hipSuccess) return e;
    const uint32_t wblocks = (n + 63) / 64;  // one wave per block: the waves spread over every CU
    e = launch_timed(prof, NPA_KERNEL_SPLIT, k_bin_place, dim3(wblocks), dim3(64), 0, stream, n,
                     (const uint32_t*)ws.keys.as<uint32_t>(), (const uint32_t*)ws.ranks.as<uint32_t>(),
                     (const uint32_t*)ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>());
    if (e != hipSuccess) return e;
    return launch_timed(prof, NPA_KERNEL_SCATTER, g.dim == 2 ? bin_scatter_for<2>(states, S) : bin_scatter_for<3>(states, S), dim3(wblocks),
                        dim3(64), 0, stream, n, (const uint32_t*)ws.keys.as<uint32_t>(),
                        (const uint32_t*)ws.bin_urow.as<uint32_t>(), (const uint32_t*)ws.bin_offsets.as<uint32_t>(),
                        (const uint32_t*)ws.tmpidx.as<uint32_t>(), (const uint32_t*)ws.totals.as<uint32_t>(),
                        (const uint32_t*)ws.bin_list.as<uint32_t>(), tpi_log2, pos, states, S, g,
                        ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(), ws.srec.as<float4>(), ws.scoord.as<int4>(),
                        ws.sstate.as<float>(), tg, ws.worklist.as<uint2>(), ws.act_rows.as<uint32_t>(),
                        ws.row_of.as<uint32_t>(), ws.dir_e.as<int4>());
}

// The two-launch build applies to a payload build of small systems whose bins are cells or
// coordinate bins (the reference's mixing-hash bins keep the four-launch build).
static bool sys_build_applies(const HashgridPlan& plan, const GridParams& g, uint32_t n) {
    return n > 0 && plan.cells <= kSysMaxCells && n <= kSysMaxRounds * kSysThreads && plan.tpi <= 64 &&
           (plan.tpi & (plan.tpi - 1)) == 0 && (g.mode != 1 || g.spatial);
}

static hipError_t launch_sys(const GridParams& g, const HashgridPlan& plan, const float4* pos, const float* states,
                             uint32_t S, uint32_t batch, uint32_t n, Workspace& ws, const SplitTargets& tg,
                             hipStream_t stream, Profiler* prof) {
    const uint32_t rounds = (n + kSysThreads - 1) / kSysThreads;
#define NPA_SYS(RR) \
    return g.dim == 2 ? launch_sys_r<2, RR>(g, plan, pos, states, S, batch, n, ws, tg, stream, prof) \
                      : launch_sys_r<3, RR>(g, plan, pos, states, S, batch, n, ws, tg, stream, prof)
    if (rounds <= 1) NPA_SYS(1);
    if (rounds <= 2) NPA_SYS(2);
    NPA_SYS(4);
#undef NPA_SYS
}

// ------------------------------------------------------------------ launch
template <int R>
static hipError_t launch_rank_r(uint32_t blocks, uint32_t waves, uint32_t lds_bytes,
                                uint32_t tiles_per_sys, uint32_t key_bits, const GridParams& g,
                                const float4* pos, const uint32_t* keys_in, const uint32_t* d_count,
                                uint32_t n, uint32_t* keys, uint32_t* ranks, uint32_t* table,
                                uint32_t* flags, uint32_t* wl_count, unsigned long long* scan_status,
                                uint32_t nstatus, hipStream_t stream, Profiler* prof, const SplitTargets& T,
                                int* tile_span, uint32_t pack) {
    if (lds_bytes > 32768) {
        static LdsLimitFlags limit;
        const hipError_t e = raise_lds_limit((const void*)k_hash_rank<R>, limit);
        if (e != hipSuccess) return e;
    }
    // the first `waves` waves rank; all of them clear the tile's counters and write its histogram
    // row, O(cells) work that wide grids (many cells per tile) spread over 16 waves
    const uint32_t threads = g.cells >= 4096 ? 1024 : 256;
    return launch_timed(prof, NPA_KERNEL_HASH_RANK, k_hash_rank<R>, dim3(blocks), dim3(threads), lds_bytes, stream,
                        pos, keys_in, d_count, n, tiles_per_sys, waves, g, key_bits, keys, ranks, table, flags,
                        wl_count, scan_status, nstatus, T, tile_span, pack);
}

static hipError_t launch_rank(uint32_t rounds, uint32_t blocks, uint32_t waves, uint32_t lds_bytes,
                              uint32_t tiles_per_sys, uint32_t key_bits, const GridParams& g,
                              const float4* pos, const uint32_t* keys_in, const uint32_t* d_count,
                              uint32_t n, uint32_t* keys, uint32_t* ranks, uint32_t* table,
                              uint32_t* flags, uint32_t* wl_count, unsigned long long* scan_status,
                              uint32_t nstatus, hipStream_t stream, Profiler* prof,
                              const SplitTargets& T = SplitTargets{}, int* tile_span = nullptr,
                              uint32_t pack = 0) {
#define NPA_RANK(RR)                                                                             \
    return launch_rank_r<RR>(blocks, waves, lds_bytes, tiles_per_sys, key_bits, g, pos, keys_in, \
                             d_count, n, keys, ranks, table, flags, wl_count, scan_status, nstatus, stream, prof, \
                             T, tile_span, pack)
    switch (rounds) {
        case 1: NPA_RANK(1);
        case 2: NPA_RANK(2);
        case 4: NPA_RANK(4);
        case 8: NPA_RANK(8);
        case 16: NPA_RANK(16);
        default: NPA_RANK(32);
    }
#undef NPA_RANK
}

hipError_t launch_hashgrid(const HashgridPlan& plan, const GridParams& g, const float4* pos,
                           const float* states, uint32_t state_dims, uint32_t batch, uint32_t n,
                           Workspace& ws, bool payload, hipStream_t stream, Profiler* prof,
                           const SplitTargets* targets) {
    const uint64_t total = (uint64_t)batch * n;
    if (payload && sys_build_applies(plan, g, n)) {
        const SplitTargets tg = targets ? *targets : SplitTargets{};
        return launch_sys(g, plan, pos, states, state_dims, batch, n, ws, tg, stream, prof);
    }
    if (payload && bin_build_applies(plan, g, batch, n)) {
        const SplitTargets tg = targets ? *targets : SplitTargets{};
        return launch_bins(plan, g, pos, states, state_dims, n, ws, tg, stream, prof);
    }
    const uint32_t kblocks = (plan.cells + 255) / 256;  // 256-key blocks of the one-pass scan
    const SplitTargets tg = targets ? *targets : SplitTargets{};
    // Folded build (one system whose bins are cells or coordinate bins): the rank kernel also counts
    // each tile's update-mask targets per key (in the table's high half) and the scatter emits what
    // the split would - its launch is saved
    // (its target counters take C u16 of LDS beside the rank counters: where both do not fit, fewer
    // waves rank the same tile in more rounds)
    // Packed (a wave ranks at most 128 particles and the system's prefixes fit 16 bits): each wave's
    // counters carry its targets too, so targets get ranks within their tile's key and the scatter
    // computes their compact rows without atomics; only the rank counters take LDS.
    uint32_t rank_waves = plan.waves, rank_rounds = plan.rounds;
    const uint32_t pack_lds = ((rank_waves * plan.cells + 1) & ~1u) * 2;
    const bool pack = rank_rounds <= 2 && n <= 65536 && pack_lds + 1024 <= kMaxLdsBytes;
    auto fold_lds_of = [&](uint32_t wv) { return ((wv * plan.cells + 1) & ~1u) * 2 + (plan.cells + 1) / 2 * 4; };
    while (!pack && fold_lds_of(rank_waves) + 1024 > kMaxLdsBytes && rank_waves > 1 && rank_rounds < 32) {
        rank_waves /= 2;
        rank_rounds *= 2;
    }
    const uint32_t fold_lds = pack ? pack_lds : fold_lds_of(rank_waves);
    const bool fold = payload && batch == 1 && (g.mode != 1 || g.spatial) && (plan.tpi & (plan.tpi - 1)) == 0 &&
                      fold_lds + 1024 <= kMaxLdsBytes;
    if (!fold) {
        rank_waves = plan.waves;
        rank_rounds = plan.rounds;
    }
    hipError_t e = launch_rank(rank_rounds, batch * plan.tiles_per_sys, rank_waves, fold ? fold_lds : plan.lds_bytes,
                               plan.tiles_per_sys, plan.key_bits, g, pos, nullptr, nullptr, n, ws.keys.as<uint32_t>(),
                               ws.ranks.as<uint32_t>(), ws.table.as<uint32_t>(), ws.flags.as<uint32_t>(),
                               ws.wl_count.as<uint32_t>(), ws.scan_status.as<unsigned long long>(),
                               2 * batch * kblocks + 1,  // the status words and the scan's ticket counter
                               stream, prof, tg, fold ? ws.tile_span.as<int>() : nullptr, fold && pack ? 1u : 0u);
    if (e != hipSuccess) return e;
    if (fold) {
        const uint32_t tpi_log2 = (uint32_t)__builtin_ctz(plan.tpi);
        e = launch_timed(prof, NPA_KERNEL_TABLE_SCAN, k_table_offsets_fold, dim3(kblocks), dim3(256), 0, stream,
                         ws.table.as<uint32_t>(), ws.bin_offsets.as<uint32_t>(),
                         ws.scan_status.as<unsigned long long>(), plan.cells, plan.tiles_per_sys, n, tpi_log2, g,
                         (const int*)ws.tile_span.as<int>(), ws.totals.as<uint32_t>(), ws.bin_list.as<uint32_t>(),
                         ws.dir_n.as<uint32_t>(), ws.wl_count.as<uint32_t>(), pack ? 1u : 0u);
        if (e != hipSuccess) return e;
        FoldOut F;
        F.item_base = ws.totals.as<uint32_t>();
        F.row_next = ws.bin_list.as<uint32_t>();
        F.worklist = ws.worklist.as<uint2>();
        F.act_rows = ws.act_rows.as<uint32_t>();
        F.row_of = ws.row_of.as<uint32_t>();
        F.dir_e = ws.dir_e.as<int4>();
        F.tpi_log2 = tpi_log2;
        F.packed = pack ? 1u : 0u;
        auto scat = g.dim == 2 ? k_scatter_payload<2> : k_scatter_payload<3>;
        const uint32_t blocks = (uint32_t)((total + 255) / 256);
        return launch_timed(prof, NPA_KERNEL_SCATTER, scat, dim3(blocks), dim3(256), 0, stream, n, (uint32_t)total,
                            plan.tile, plan.tiles_per_sys, plan.cells, ws.keys.as<uint32_t>(), ws.ranks.as<uint32_t>(),
                            ws.table.as<uint32_t>(), ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>(),
                            ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(), pos, states, state_dims, g,
                            ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(), tg,
                            ws.flags.as<uint32_t>(), F);
    }
    if (batch >= 8 && plan.cells <= 4096 && plan.tiles_per_sys <= 4) {  // many small systems: a block each
        auto k = plan.cells <= 1024 ? k_table_offsets_sys<1, 4> : k_table_offsets_sys<4, 4>;
        e = launch_timed(prof, NPA_KERNEL_TABLE_SCAN, k, dim3(batch), dim3(1024), 0, stream, ws.table.as<uint32_t>(),
                         ws.bin_offsets.as<uint32_t>(), plan.cells, plan.tiles_per_sys, n, batch);
    } else {
        e = launch_timed(prof, NPA_KERNEL_TABLE_SCAN, k_table_offsets_scan, dim3(kblocks, batch), dim3(256), 0, stream,
                         ws.table.as<uint32_t>(), ws.bin_offsets.as<uint32_t>(),
                         ws.scan_status.as<unsigned long long>(), plan.cells, plan.tiles_per_sys, n, batch);
    }
    if (e != hipSuccess) return e;
    const uint32_t blocks = (uint32_t)((total + 255) / 256);
    if (!payload)
        return launch_timed(prof, NPA_KERNEL_SCATTER, k_scatter, dim3(blocks), dim3(256), 0, stream, n,
                            (uint32_t)total, plan.tile, plan.tiles_per_sys, plan.cells, ws.keys.as<uint32_t>(),
                            ws.ranks.as<uint32_t>(), ws.table.as<uint32_t>(), ws.bin_offsets.as<uint32_t>(),
                            ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(), ws.flags.as<uint32_t>());
    auto scat = g.dim == 2 ? k_scatter_payload<2> : k_scatter_payload<3>;
    e = launch_timed(prof, NPA_KERNEL_SCATTER, scat, dim3(blocks), dim3(256), 0, stream, n, (uint32_t)total,
                     plan.tile, plan.tiles_per_sys, plan.cells, ws.keys.as<uint32_t>(), ws.ranks.as<uint32_t>(),
                     ws.table.as<uint32_t>(), ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>(),
                     ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(), pos, states, state_dims, g, ws.srec.as<float4>(),
                     ws.scoord.as<int4>(), ws.sstate.as<float>(), tg, ws.flags.as<uint32_t>(), FoldOut{});
    if (e != hipSuccess) return e;
    const uint32_t nbins = batch * plan.cells;
    auto split = g.dim == 2 ? k_split<2> : k_split<3>;
    if ((uint64_t)nbins * 4 <= total) {  // dense bins: a wave per bin
        const uint32_t sblocks = (nbins + kSplitWaves - 1) / kSplitWaves;
        return launch_timed(prof, NPA_KERNEL_SPLIT, split, dim3(sblocks), dim3(64 * kSplitWaves), 0, stream, pos,
                            states, state_dims, n, nbins, g, ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>(),
                            ws.perm.as<uint32_t>(), ws.inv.as<uint32_t>(), ws.srec.as<float4>(),
                            ws.scoord.as<int4>(), ws.sstate.as<float>(), ws.dir_n.as<uint32_t>(),
                            ws.dir_e.as<int4>(), ws.worklist.as<uint2>(), ws.wl_count.as<uint32_t>(), plan.tpi, tg,
                            ws.act_rows.as<uint32_t>(), ws.row_of.as<uint32_t>(), (const uint32_t*)nullptr,
                            (const uint32_t*)nullptr);
    }
    // sparse bins: one lane per small bin, then a wave per listed (larger) bin; a listed bin holds
    // more than kThinMax particles, so at most total / (kThinMax + 1) bins are listed
    ProfScope ps(prof, NPA_KERNEL_SPLIT, stream);  // both kernels count as the step's one split
    auto thin = g.dim == 2 ? k_split_thin<2> : k_split_thin<3>;
    hipLaunchKernelGGL(thin, dim3((nbins + kThinThreads - 1) / kThinThreads), dim3(kThinThreads), 0, stream, pos, states, state_dims, n, nbins, g,
                       ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>(), ws.perm.as<uint32_t>(),
                       ws.inv.as<uint32_t>(), ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(),
                       ws.dir_n.as<uint32_t>(), ws.dir_e.as<int4>(), ws.worklist.as<uint2>(),
                       ws.wl_count.as<uint32_t>(), plan.tpi, tg, ws.act_rows.as<uint32_t>(), ws.row_of.as<uint32_t>(),
                       ws.bin_list.as<uint32_t>());
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const uint64_t listed_max = total / (kThinMax + 1);
    const uint32_t sblocks = (uint32_t)std::max<uint64_t>(1, (listed_max + kSplitWaves - 1) / kSplitWaves);
    hipLaunchKernelGGL(split, dim3(sblocks), dim3(64 * kSplitWaves), 0, stream, pos, states, state_dims, n, nbins, g,
                       ws.bin_offsets.as<uint32_t>(), ws.tmpidx.as<uint32_t>(), ws.perm.as<uint32_t>(),
                       ws.inv.as<uint32_t>(), ws.srec.as<float4>(), ws.scoord.as<int4>(), ws.sstate.as<float>(),
                       ws.dir_n.as<uint32_t>(), ws.dir_e.as<int4>(), ws.worklist.as<uint2>(),
                       ws.wl_count.as<uint32_t>(), plan.tpi, tg, ws.act_rows.as<uint32_t>(), ws.row_of.as<uint32_t>(),
                       (const uint32_t*)ws.bin_list.as<uint32_t>(), (const uint32_t*)(ws.wl_count.as<uint32_t>() + kListedWord));
    return hipGetLastError();
}

// ------------------------------------------------------ generic key sort
__global__ __launch_bounds__(256) void k_scatter_vals(const uint32_t* __restrict__ keys,
                                                      const uint32_t* __restrict__ vals,
                                                      const uint32_t* __restrict__ d_count,
                                                      uint32_t cap, uint32_t tile, uint32_t C,
                                                      const uint32_t* __restrict__ ranks,
                                                      const uint32_t* __restrict__ table,
                                                      const uint32_t* __restrict__ offsets,
                                                      uint32_t* __restrict__ out_vals) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t dc = *d_count;
    const uint32_t count = dc < cap ? dc : cap;
    if (i >= count) return;
    const uint32_t key = keys[i];
    const uint32_t dst = offsets[key] + table[(uint64_t)(i / tile) * C + key] + ranks[i];
    out_vals[dst] = vals ? vals[i] : i;
}

bool make_key_sort_plan(uint32_t cap, uint32_t C, HashgridPlan* p) {
    if (C == 0 || C > 65536) return false;
    p->cells = C;
    p->key_bits = C <= 1 ? 0 : 32 - __builtin_clz(C - 1);
    p->waves = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(4, 32768 / C));
    p->lds_bytes = p->waves * C * 2;
    const uint64_t budget = std::max<uint64_t>(2 * (uint64_t)cap, C);
    uint32_t rounds = 1;
    while (rounds < 32) {
        uint64_t tile = (uint64_t)p->waves * rounds * 64;
        if (((cap + tile - 1) / tile) * (uint64_t)C <= budget) break;
        rounds *= 2;
    }
    // The table scan walks tiles_per_sys entries of each bin serially: with few bins (screen
    // tiles) prefer fewer, larger rank tiles.
    while (rounds < 32 && (cap + (uint64_t)p->waves * rounds * 64 - 1) / ((uint64_t)p->waves * rounds * 64) > 256)
        rounds *= 2;
    p->rounds = rounds;
    p->tile = p->waves * rounds * 64;
    p->tiles_per_sys = std::max<uint32_t>(1, (cap + p->tile - 1) / p->tile);
    p->table_entries = (uint64_t)p->tiles_per_sys * C;
    return true;
}

hipError_t launch_key_sort(const HashgridPlan& p, const uint32_t* keys, const uint32_t* vals,
                           const uint32_t* d_count, uint32_t cap, uint32_t* ranks, uint32_t* table,
                           uint32_t* totals, uint32_t* offsets, uint32_t* out_vals, uint32_t* flags,
                           hipStream_t stream) {
    GridParams g{};
    g.cells = p.cells;
    hipError_t e = launch_rank(p.rounds, p.tiles_per_sys, p.waves, p.lds_bytes, p.tiles_per_sys,
                               p.key_bits, g, nullptr, keys, d_count, cap, nullptr, ranks, table,
                               flags, nullptr, nullptr, 0u, stream, nullptr);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_table_scan, dim3((p.cells + 255) / 256, 1), dim3(256), 0, stream, table, totals,
                       p.cells, p.tiles_per_sys);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = launch_offsets_scan(totals, offsets, p.cells, cap, 1u, stream, nullptr)) != hipSuccess) return e;
    if (cap == 0) return hipSuccess;
    hipLaunchKernelGGL(k_scatter_vals, dim3((cap + 255) / 256), dim3(256), 0, stream, keys, vals, d_count,
                       cap, p.tile, p.cells, ranks, table, offsets, out_vals);
    return hipGetLastError();
}

int device_cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

}  // namespace npa
