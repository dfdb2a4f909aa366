// sort_and_bin on gfx950: per-image depth range, packed-key emission, a stable LSD radix sort,
// and tile bin edges. Restates splax/_rasterize/_sort/_sort.py:29-171 and
// splax/_rasterize/_sort/_kernels.py:28-153,214-241; the sort replaces warp-lang's
// radix_sort_pairs (called at splax/_rasterize/_sort/_sort.py:136).
//
// Sort design: each pass is reduce-then-scan over partitions of 4096 to 8192 keys: (1) every
// partition counts its digits, (2) one workgroup per digit scans that digit's counts over the
// partitions and writes the digit's total, (3) every partition ranks its keys stably with
// ballot-based digit matching per wave and scatters keys and values through LDS so that each
// digit's run (about 32 keys) leaves as a contiguous write; each XCD counts and scatters one
// contiguous segment of the partitions, so the runs and counts that neighbouring partitions
// write side by side merge in one L2. No partition waits on another: on MI355X the eight XCDs
// have separate L2s, so the per-digit status polling of a single-pass (look-back) sort costs
// device-scope round trips and partial-line writes that the extra count read does not. Ranking
// follows position order (wave-striped items, lanes in order, waves in order, partitions in
// index order), so the sort is stable: ties keep emission order, which is the reference's
// (key, position) order.
//
// Each key carries two values: the reference's value (the flat item id) and the key's emission
// position. The positions let the backward blend store each intersection's gradient in emission
// order, where every item's intersections are contiguous; a forward that no backward follows
// sorts without them. Packed keys leave the pass over bits 8-15 as their 16-bit high halves
// (image and tile fields), which the last two passes and the bin edges move, unless the caller
// returns the sorted keys. A capacity-bounded caller need not know the count: the kernels then
// read it from device memory (live_count) and the grids cover the capacity.
#include "splat_common.hpp"
#include "splat_internal.hpp"

namespace splat {

// The intersection count a sort kernel works on: `bound` when the host knows the count (m_dev
// null), else the count the projection left in device memory clamped to [0, bound], where bound
// is the caller's list capacity (a count above it, or a wrapped negative one, is reported by the
// host once the call's launches are queued; the kernels meanwhile stay inside the buffers).
__device__ __forceinline__ int64_t live_count(const int32_t* m_dev, int64_t bound) {
    if (!m_dev) return bound;
    const int64_t m = *m_dev;
    return m < 0 ? 0 : (m > bound ? bound : m);
}

// ------------------------------------------------------------------ depth range
// _depth_minmax, splax/_rasterize/_sort/_kernels.py:38-73: per-image [dmin, dmax] over items with
// radii > 0. Stage 1 writes one partial per workgroup; stage 2 (one workgroup per image) folds
// them. Floats are mapped to order-preserving unsigned integers for the reductions.

constexpr int kMmThreads = 256;
constexpr int kMmItems = 16;


__global__ void __launch_bounds__(kMmThreads)
minmax_partial_kernel(const float* depths, const int32_t* radii, int32_t n,
                      int32_t blocks_per_image, uint32_t* partial) {
    __shared__ uint32_t s_lo[kMmThreads / 64], s_hi[kMmThreads / 64];
    const int image = blockIdx.y;
    const int64_t base = (int64_t)image * n + (int64_t)blockIdx.x * (kMmThreads * kMmItems);
    const int64_t end = (int64_t)image * n + n;
    uint32_t lo = 0xffffffffu, hi = 0u;
    // both arrays are loaded for every item (not the depth behind the radius test), so all the
    // loads of a thread are in flight together
#pragma unroll
    for (int k = 0; k < kMmItems; ++k) {
        const int64_t idx = base + (int64_t)k * kMmThreads + threadIdx.x;
        const bool in = idx < end;
        const int32_t r = in ? radii[idx] : 0;
        const float d = in ? depths[idx] : 0.0f;
        if (r > 0) {
            const uint32_t o = f2ord(d);
            lo = o < lo ? o : lo;
            hi = o > hi ? o : hi;
        }
    }
    // the wave's range in lane 63 (DPP; every lane is active here)
    lo = wave_minmax_to_lane63<false>(lo);
    hi = wave_minmax_to_lane63<true>(hi);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 63) {
        s_lo[wave] = lo;
        s_hi[wave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        lo = 0xffffffffu;
        hi = 0u;
        for (int w = 0; w < kMmThreads / 64; ++w) {
            lo = s_lo[w] < lo ? s_lo[w] : lo;
            hi = s_hi[w] > hi ? s_hi[w] : hi;
        }
        int64_t slot = (int64_t)image * blocks_per_image + blockIdx.x;
        partial[2 * slot] = lo;
        partial[2 * slot + 1] = hi;
    }
}

// Stage 2.
__global__ void __launch_bounds__(kMmThreads)
minmax_final_kernel(const uint32_t* partial, int32_t blocks_per_image, float* mm) {
    __shared__ uint32_t s_lo[kMmThreads / 64], s_hi[kMmThreads / 64];
    const int image = blockIdx.x;
    uint32_t lo = 0xffffffffu, hi = 0u;
    for (int b = threadIdx.x; b < blocks_per_image; b += kMmThreads) {
        int64_t slot = (int64_t)image * blocks_per_image + b;
        uint32_t a = partial[2 * slot], c = partial[2 * slot + 1];
        lo = a < lo ? a : lo;
        hi = c > hi ? c : hi;
    }
    // the wave's range in lane 63 (DPP; every lane is active here)
    lo = wave_minmax_to_lane63<false>(lo);
    hi = wave_minmax_to_lane63<true>(hi);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 63) {
        s_lo[wave] = lo;
        s_hi[wave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        lo = 0xffffffffu;
        hi = 0u;
        for (int w = 0; w < kMmThreads / 64; ++w) {
            lo = s_lo[w] < lo ? s_lo[w] : lo;
            hi = s_hi[w] > hi ? s_hi[w] : hi;
        }
        // no visible item: the reference's +-1e30 seeds remain (drange < 0 -> depth_q = 0)
        mm[2 * image] = hi == 0u ? 1.0e30f : ord2f(lo);
        mm[2 * image + 1] = hi == 0u ? -1.0e30f : ord2f(hi);
    }
}

// ------------------------------------------------------------------ key emission
// _map_intersects_32bit, splax/_rasterize/_sort/_kernels.py:76-153

struct EmitParams {
    const float* xys; const float* depths; const int32_t* radii; const float* conics;
    const float* map_opac; int64_t rows_map_opac;
    const int32_t* cum; const float* mm;
    int32_t n; int64_t total; int64_t M;
    const int32_t* m_dev;  // device-resident count (live_count), or null: M is the count
    // the render path: cum is chunk-local, finalized here (cum_fix, the same array) from each
    // chunk's exclusive prefix; nth holds the items' own counts
    const uint32_t* chunk_prefix; const int32_t* nth; int32_t* cum_fix;
    int32_t tiles_x, tiles_y, tile_bits, depth_bits;
    void* keys; int32_t* owner;
};

// kWide: the 64-bit key of _map_intersects_64bit (splax/_rasterize/_sort/_kernels.py:156-211),
// (image << (32 + tile_bits)) | (tile << 32) | the depth's raw float bits (int32, widened with
// sign extension). Otherwise the packed key image | tile | quantized depth.
template <bool kWide>
__global__ void __launch_bounds__(256) emit_keys_kernel(EmitParams P) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= P.total) return;
    // Every input of the item is loaded first, culled items included: behind the radius test,
    // or behind the store of the final prefix (which the compiler cannot prove disjoint from
    // them), each group of loads was one more dependent memory round trip per item (config 3's
    // emission 0.139 ms that way against 0.117 ms).
    const int32_t bid = (int32_t)(idx / P.n);
    int32_t fin_raw = 0, nth = 0;
    int64_t cur;
    if (P.chunk_prefix) {
        fin_raw = P.cum_fix[idx];
        nth = P.nth[idx];
    }
    const uint32_t cpre = P.chunk_prefix ? P.chunk_prefix[idx / kProjChunkItems] : 0u;
    const int32_t prev = (!P.chunk_prefix && idx > 0) ? P.cum[idx - 1] : 0;
    const int32_t rad = P.radii[idx];
    const float depth = P.depths[idx];
    const float2 c = reinterpret_cast<const float2*>(P.xys)[idx];
    const float ca = P.conics[3 * idx], cb = P.conics[3 * idx + 1], cc = P.conics[3 * idx + 2];
    const float opac = P.map_opac[idx % P.rows_map_opac];
    float dmin = 0.0f, dmax = 0.0f;
    if constexpr (!kWide) {
        dmin = P.mm[2 * bid];
        dmax = P.mm[2 * bid + 1];
    }
    if (P.chunk_prefix) {
        // every item's final inclusive prefix (an output of the call), and the start of its
        // keys as that prefix less its own count: each thread reads and writes its own entry
        // only. Unsigned adds keep cum_tiles_hit's int32 wrap-around.
        const uint32_t fin = (uint32_t)fin_raw + cpre;
        P.cum_fix[idx] = (int32_t)fin;
        cur = (int32_t)(fin - (uint32_t)nth);
    } else {
        cur = prev;
    }
    if (rad <= 0) return;
    // a consistent (radii, conics, cum) never leaves [0, M); inconsistent inputs stop here
    if (cur < 0) return;
    const int64_t M = live_count(P.m_dev, P.M);
    int32_t dq = 0, iid_enc = 0;
    uint64_t wide_base = 0;
    if constexpr (kWide) {
        const int64_t depth_id = (int64_t)__float_as_int(depth);
        wide_base = ((uint64_t)(uint32_t)bid << (32 + P.tile_bits)) | (uint64_t)depth_id;
    } else {
        const float drange = dmax - dmin;
        const int32_t qmax = (1 << P.depth_bits) - 1;
        const float maxq = (float)qmax;
        if (drange > 0.0f) {
            float f = (depth - dmin) / drange;
            dq = iminw(imaxw(f2i(f * maxq), 0), qmax);
        }
        iid_enc = (int32_t)((uint32_t)bid << (P.depth_bits + P.tile_bits));
    }
    const float t = iso_level(opac);
    Ellipse e = ellipse_init(ca, cb, cc, t, c.x, c.y, P.tiles_x, P.tiles_y);
    if (!e.valid) return;
    float I0, I1;
    ellipse_init_span(e, I0, I1);
    for (int32_t u = e.rmin0; u < e.rmax0; ++u) {
        int32_t mn, mx;
        ellipse_column(e, u, I0, I1, mn, mx);
        for (int32_t v = mn; v < mx; ++v) {
            if (cur >= M) return;
            int32_t tile_id = e.isY ? u * P.tiles_x + v : v * P.tiles_x + u;
            if constexpr (kWide)
                static_cast<uint64_t*>(P.keys)[cur] =
                    wide_base | ((uint64_t)(uint32_t)tile_id << 32);
            else
                static_cast<int32_t*>(P.keys)[cur] = iid_enc | (tile_id << P.depth_bits) | dq;
            P.owner[cur] = (int32_t)idx;
            ++cur;
        }
    }
}

// The digits a sort visits: 8-bit digits at these shifts (packed key: 0, 8, 16, 24).
struct PassShifts {
    int32_t n;
    int32_t shift[kMaxPasses];
};

// ------------------------------------------------------------------ reduce-then-scan passes

constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
static_assert(kSortThreads * 4 == kSortTileMin, "smallest partition");

// The partition that workgroup blockIdx.x of a count or scatter launch takes, or -1 for none.
// Workgroup b runs on XCD b mod 8 (the dispatcher deals workgroups to the eight XCDs in turn).
// Each XCD takes one contiguous segment of the live partitions, in order, so neighbouring
// partitions share an L2: the runs of one digit that they scatter side by side, and the counts
// they store side by side in a digit's row, merge there into whole lines before they leave it
// (dealt in turn, neighbouring partitions sit on different XCDs and every run end or count
// leaves its L2 as a partial-line write). The segments split the live partitions, not the grid,
// which a capacity-bounded caller sizes above the count, so every XCD gets an equal share. The
// grid must hold at least 8 * ceil(live_parts / 8) workgroups.
__device__ __forceinline__ int64_t xcd_segment_part(int64_t live_parts) {
    const int64_t per_xcd = (live_parts + 7) >> 3;
    const int64_t seg_pos = blockIdx.x >> 3;
    if (seg_pos >= per_xcd) return -1;
    const int64_t part = (int64_t)(blockIdx.x & 7u) * per_xcd + seg_pos;
    return part < live_parts ? part : -1;
}

// Workgroups of a count or scatter launch over `parts` partitions: whole groups of eight, one
// workgroup per XCD (the kernels deal the live partitions to XCD segments).
static unsigned segment_grid(int64_t parts) { return (unsigned)((parts + 7) / 8 * 8); }

// (1) digit counts of one partition of kItems * kSortThreads keys, stored digit-major:
// counts[d * parts + p]. The first pass also clears the tile bins (nbins2 > 0). Only the live
// partitions store counts; the digit scan reads the columns past them as zero.
template <typename K, int kItems>
__global__ void __launch_bounds__(kSortThreads)
rts_count_kernel(const K* __restrict__ keys, int64_t M_bound, const int32_t* __restrict__ m_dev,
                 int shift, uint32_t* __restrict__ counts, int64_t parts,
                 int32_t* __restrict__ bins, int64_t nbins2) {
    __shared__ uint32_t s_h[kSortWaves][256];
    const int tid = threadIdx.x, wave = tid >> 6;
    for (int i = tid; i < kSortWaves * 256; i += kSortThreads) (&s_h[0][0])[i] = 0u;
    // tile bins start at (0, 0): the bin-edge launch writes only tiles that own intersections
    for (int64_t i = (int64_t)blockIdx.x * kSortThreads + tid; i < nbins2;
         i += (int64_t)gridDim.x * kSortThreads)
        bins[i] = 0;
    __syncthreads();
    const int64_t M = live_count(m_dev, M_bound);
    constexpr int64_t kPart = (int64_t)kItems * kSortThreads;
    const int64_t part = xcd_segment_part((M + kPart - 1) / kPart);
    if (part < 0) return;  // uniform, after the workgroup's share of the bin clearing
    const int64_t base = part * kPart;
    K key[kItems];
    constexpr int kBytes = kItems * (int)sizeof(K);
    const int64_t my0 = base + (int64_t)tid * kItems;
    if constexpr (sizeof(K) <= 4 && kBytes % 4 == 0) {
        // a digit count does not depend on the keys' order: each thread takes kItems
        // consecutive keys, read as whole 32-bit words (the run starts kBytes * tid bytes into
        // the partition, so the widest load that divides kBytes is aligned), where one load per
        // key took more load instructions than the bytes need (the sort 0.106 -> 0.103 ms at
        // config 2, 0.715 -> 0.692 ms at config 4); 64-bit keys and odd 16-bit runs keep the
        // wave-striped scalar loads
        if (my0 + kItems <= M) {
            constexpr int kW = kBytes / 4;
            uint32_t w[kW];
            const char* src = reinterpret_cast<const char*>(keys + my0);
            if constexpr (kBytes % 16 == 0) {
#pragma unroll
                for (int q = 0; q < kW / 4; ++q) {
                    const uint4 v = reinterpret_cast<const uint4*>(src)[q];
                    w[4 * q] = v.x; w[4 * q + 1] = v.y; w[4 * q + 2] = v.z; w[4 * q + 3] = v.w;
                }
            } else if constexpr (kBytes % 8 == 0) {
#pragma unroll
                for (int q = 0; q < kW / 2; ++q) {
                    const uint2 v = reinterpret_cast<const uint2*>(src)[q];
                    w[2 * q] = v.x; w[2 * q + 1] = v.y;
                }
            } else {
#pragma unroll
                for (int q = 0; q < kW; ++q) w[q] = reinterpret_cast<const uint32_t*>(src)[q];
            }
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                if constexpr (sizeof(K) == 4)
                    key[i] = (K)w[i];
                else
                    key[i] = (K)((w[i / 2] >> (16 * (i & 1))) & 0xffffu);
            }
#pragma unroll
            for (int i = 0; i < kItems; ++i)
                atomicAdd(&s_h[wave][(uint32_t)(key[i] >> shift) & 255u], 1u);
        } else {
#pragma unroll
            for (int i = 0; i < kItems; ++i) key[i] = my0 + i < M ? keys[my0 + i] : (K)0;
#pragma unroll
            for (int i = 0; i < kItems; ++i)
                if (my0 + i < M) atomicAdd(&s_h[wave][(uint32_t)(key[i] >> shift) & 255u], 1u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int64_t pos = base + i * kSortThreads + tid;
            key[i] = pos < M ? keys[pos] : (K)0;
        }
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int64_t pos = base + i * kSortThreads + tid;
            if (pos < M) atomicAdd(&s_h[wave][(uint32_t)(key[i] >> shift) & 255u], 1u);
        }
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) c += s_h[w][tid];
        counts[(int64_t)tid * parts + part] = c;
    }
}

// Exclusive scan of one value per thread over the first 256 threads (waves 0-3) of the
// workgroup; every thread of the workgroup must call it.
__device__ __forceinline__ uint32_t scan_256(uint32_t v, uint32_t* s_tmp, uint32_t* total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t incl = (uint32_t)wave_inclusive_scan_i32((int32_t)v, lane);
    if (lane == 63 && wave < 4) s_tmp[wave] = incl;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t x = s_tmp[w];
        if (w < wave) off += x;
        tot += x;
    }
    if (total) *total = tot;
    __syncthreads();
    return off + incl - v;
}

// (2) one workgroup per digit d: counts[d][p] <- sum_{q < p} counts[d][q], and totals[d]. Four
// counts per thread: with 1024 threads up to 4096 partitions (16M keys at 4 keys per thread, 32M
// at 8) in one pass over the row. Columns past the live partitions (of part_keys keys each) count as zero.
// kThreads: 1024, or 256 when the row holds at most 1024 partitions (config 2 has 434: a
// quarter of the threads then carry counts, and the smaller workgroup's barriers are shorter;
// the sort 0.107 -> 0.106 ms).
template <int kThreads>
__global__ void __launch_bounds__(kThreads)
rts_scan_kernel(uint32_t* __restrict__ counts, int64_t parts, uint32_t* __restrict__ totals,
                int64_t M_bound, const int32_t* __restrict__ m_dev, int64_t part_keys) {
    constexpr int kScanThreads = kThreads;
    __shared__ uint32_t s_wave[kScanThreads / 64];
    const int d = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t carry = 0;
    uint32_t* row = counts + (int64_t)d * parts;
    const int64_t live = (live_count(m_dev, M_bound) + part_keys - 1) / part_keys;
    for (int64_t p0 = 0; p0 < parts; p0 += 4 * kScanThreads) {
        // four consecutive counts per thread
        const int64_t p = p0 + 4 * (int64_t)tid;
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = p + k < live ? row[p + k] : 0u;
        const uint32_t mine = (v[0] + v[1]) + (v[2] + v[3]);
        const uint32_t incl = (uint32_t)wave_inclusive_scan_i32((int32_t)mine, lane);
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        uint32_t before = carry, tot = carry;
#pragma unroll
        for (int w = 0; w < kScanThreads / 64; ++w) {
            const uint32_t x = s_wave[w];
            before += w < wave ? x : 0u;
            tot += x;
        }
        uint32_t run = before + incl - mine;  // exclusive prefix of this thread's first count
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (p + k < parts) row[p + k] = run;
            run += v[k];
        }
        carry = tot;
        __syncthreads();  // s_wave is rewritten by the next round
    }
    if (tid == 0) totals[d] = carry;
}

// (3) Stable scatter of one partition. A key of digit d at partition-local sorted slot j goes
// to (keys with a smaller digit) + offsets[d][p] + (j - first slot of d). The first pass
// generates the emission positions (vals_in == nullptr gives value = position) and reads the
// items in emission order, so no pass gathers at random; vals_out == nullptr moves no positions
// (a forward whose lists no backward reads). K is the key word (uint32_t for the
// packed key, uint64_t for the 64-bit key, ordered as unsigned). KO is the key word written:
// K, or uint16_t from uint32_t keys, the key's high half (the pass that sorts bits 8-15 of a
// packed key leaves only bits 16-30 to sort and to bin, and a packed key's depth field is at
// least 16 bits wide, so the image and tile fields sit in that half).
template <typename K, int kItems, typename KO = K>
// at most 64 VGPRs (eight waves per SIMD), so two 1024-thread workgroups share a CU
__global__ void __launch_bounds__(kSortThreads, 8)
rts_scatter_kernel(const K* __restrict__ keys_in, const int32_t* __restrict__ vals_in,
                   const int32_t* __restrict__ ids_in, KO* __restrict__ keys_out,
                   int32_t* __restrict__ vals_out, int32_t* __restrict__ ids_out,
                   int64_t M_bound, const int32_t* __restrict__ m_dev, int shift,
                   const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ totals,
                   int64_t parts) {
    constexpr int kTile = kItems * kSortThreads;
    static_assert(sizeof(KO) == sizeof(K) || (sizeof(K) == 4 && sizeof(KO) == 2),
                  "narrowing writes a 32-bit key's high half");
    // one staging buffer carries keys, then positions, then ids (three rounds), so two
    // 1024-thread workgroups fit a CU's LDS at eight keys per thread
    constexpr int kStageWords = kTile * (sizeof(K) > 4 ? (int)(sizeof(K) / 4) : 1);
    __shared__ __attribute__((aligned(16))) uint32_t s_stage[kStageWords];
    K* const s_keys = reinterpret_cast<K*>(s_stage);
    uint32_t* const s_u32 = s_stage;
    __shared__ uint32_t s_cnt[kSortWaves][256];
    __shared__ uint32_t s_local_start[256];
    __shared__ int32_t s_dest_base[256];
    __shared__ uint32_t s_tmp[4];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t M = live_count(m_dev, M_bound);
    const int64_t part = xcd_segment_part((M + kTile - 1) / kTile);
    if (part < 0) return;  // uniform, before any barrier
    const int64_t base = part * kTile;
    for (int i = tid; i < kSortWaves * 256; i += kSortThreads) (&s_cnt[0][0])[i] = 0u;
    __syncthreads();
    const int64_t wbase = base + (int64_t)wave * (kItems * 64);

    // the keys first; positions and ids are loaded a round ahead of their own LDS round, so the
    // ranking runs with only keys and ranks live
    // item i of this thread sits at my0 + 64 i (in range while 64 i < rem): one base address and
    // immediate offsets for every load
    const int64_t my0 = wbase + lane;
    const int64_t rem = M - my0;
    K key[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) key[i] = i * 64 < rem ? keys_in[my0 + i * 64] : (K)~(K)0;
    const uint32_t total_d = tid < 256 ? totals[tid] : 0u;
    const uint32_t offset_d = tid < 256 ? offsets[(int64_t)tid * parts + part] : 0u;

    // stable per-wave ranking: lanes with equal digits found by 8 ballots
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint32_t rank[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const uint32_t d = (uint32_t)(key[i] >> shift) & 255u;
        uint64_t peers = ~0ull;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        const uint32_t below = (uint32_t)__popcll(peers & lt_mask);
        const uint32_t old = s_cnt[wave][d];
        rank[i] = old + below;
        if (below == 0) s_cnt[wave][d] = old + (uint32_t)__popcll(peers);
    }
    __syncthreads();

    // per digit (thread = digit): wave offsets, local digit starts, global destinations
    uint32_t tot = 0;
    if (tid < 256) {
        // exclusive running sum over the waves, in place (one value live)
        for (int w = 0; w < kSortWaves; ++w) {
            const uint32_t c = s_cnt[w][tid];
            s_cnt[w][tid] = tot;
            tot += c;
        }
    }
    const uint32_t local_start = scan_256(tot, s_tmp, nullptr);
    const uint32_t digit_base = scan_256(total_d, s_tmp, nullptr);
    if (tid < 256) {
        s_local_start[tid] = local_start;
        s_dest_base[tid] = (int32_t)((int64_t)digit_base + offset_d - local_start);
    }
    __syncthreads();

    // partition-sorted slot of each of this thread's keys
    uint32_t slot[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const uint32_t dd = (uint32_t)(key[i] >> shift) & 255u;
        slot[i] = s_local_start[dd] + s_cnt[wave][dd] + rank[i];
    }
    const bool with_pos = vals_out != nullptr;  // uniform
    uint32_t val[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i)
        val[i] = with_pos && i * 64 < rem ? (vals_in ? (uint32_t)vals_in[my0 + i * 64]
                                                     : (uint32_t)(my0 + i * 64))
                                          : 0u;
    // round 1, keys. Each digit's run is contiguous in the output, so consecutive j write
    // consecutive addresses; the destinations are kept for the other two rounds.
#pragma unroll
    for (int i = 0; i < kItems; ++i) s_keys[slot[i]] = key[i];
    __syncthreads();
    const int64_t valid = (M - base) < kTile ? (M - base) : kTile;
    // the digit of output slot r * kSortThreads + tid, four to a register: rounds 2 and 3 take the
    // destination from s_dest_base again
    uint32_t dig[(kItems + 3) / 4] = {};
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
        const int j = r * kSortThreads + tid;
        if (j < valid) {
            const K k = s_keys[j];
            const uint32_t d = (uint32_t)(k >> shift) & 255u;
            dig[r >> 2] |= d << (8 * (r & 3));
            if constexpr (sizeof(KO) < sizeof(K))
                keys_out[s_dest_base[d] + j] = (KO)(k >> 16);
            else
                keys_out[s_dest_base[d] + j] = k;
        }
    }
    __syncthreads();
    // round 2, emission positions
    uint32_t gid[kItems];
    if (with_pos) {
#pragma unroll
        for (int i = 0; i < kItems; ++i) s_u32[slot[i]] = val[i];
    }
#pragma unroll
    for (int i = 0; i < kItems; ++i) gid[i] = i * 64 < rem ? (uint32_t)ids_in[my0 + i * 64] : 0u;
    if (with_pos) {
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kItems; ++r) {
            const int j = r * kSortThreads + tid;
            if (j < valid)
                vals_out[s_dest_base[(dig[r >> 2] >> (8 * (r & 3))) & 255u] + j] =
                    (int32_t)s_u32[j];
        }
        __syncthreads();
    }
    // round 3, item ids
#pragma unroll
    for (int i = 0; i < kItems; ++i) s_u32[slot[i]] = gid[i];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kItems; ++r) {
        const int j = r * kSortThreads + tid;
        if (j < valid)
            ids_out[s_dest_base[(dig[r >> 2] >> (8 * (r & 3))) & 255u] + j] = (int32_t)s_u32[j];
    }
}

// One pass of the sort: count, scan, scatter with kItems keys per thread.
template <typename K, int kItems, typename KO = K>
static void launch_pass(const K* keys_in, const int32_t* vals_in, const int32_t* ids_in,
                        KO* keys_out, int32_t* vals_out, int32_t* ids_out, int64_t M,
                        const int32_t* m_dev, int shift, uint32_t* counts, uint32_t* totals,
                        int32_t* bins, int64_t nbins2, hipStream_t stream) {
    // M bounds the count (live_count): the grid covers M keys
    const int64_t parts = (M + (int64_t)kItems * kSortThreads - 1) / ((int64_t)kItems * kSortThreads);
    hipLaunchKernelGGL((rts_count_kernel<K, kItems>), dim3(segment_grid(parts)),
                       dim3(kSortThreads), 0, stream, keys_in, M, m_dev, shift, counts, parts,
                       bins, nbins2);
    if (parts <= 4 * 256)
        hipLaunchKernelGGL(rts_scan_kernel<256>, dim3(256), dim3(256), 0, stream, counts, parts,
                           totals, M, m_dev, (int64_t)kItems * kSortThreads);
    else
        hipLaunchKernelGGL(rts_scan_kernel<1024>, dim3(256), dim3(1024), 0, stream, counts,
                           parts, totals, M, m_dev, (int64_t)kItems * kSortThreads);
    hipLaunchKernelGGL((rts_scatter_kernel<K, kItems, KO>), dim3(segment_grid(parts)),
                       dim3(kSortThreads), 0, stream, keys_in, vals_in, ids_in, keys_out,
                       vals_out, ids_out, M, m_dev, shift, counts, totals, parts);
}

// A pass over packed keys of one of three forms: 32-bit keys in and out (kind 0), 32-bit in and
// their high halves out (kind 1), 16-bit high halves in and out (kind 2; shift counts from bit
// 16).
template <int kItems>
static void packed_pass(int kind, const void* ki, const int32_t* vin, const int32_t* gin,
                        void* ko, int32_t* vout, int32_t* iout, int64_t M, const int32_t* m_dev,
                        int shift, uint32_t* counts, uint32_t* totals, int32_t* bins,
                        int64_t nb2, hipStream_t stream) {
    if (kind == 0)
        launch_pass<uint32_t, kItems>(static_cast<const uint32_t*>(ki), vin, gin,
                                      static_cast<uint32_t*>(ko), vout, iout, M, m_dev, shift,
                                      counts, totals, bins, nb2, stream);
    else if (kind == 1)
        launch_pass<uint32_t, kItems, uint16_t>(static_cast<const uint32_t*>(ki), vin, gin,
                                                static_cast<uint16_t*>(ko), vout, iout, M, m_dev,
                                                shift, counts, totals, bins, nb2, stream);
    else
        launch_pass<uint16_t, kItems>(static_cast<const uint16_t*>(ki), vin, gin,
                                      static_cast<uint16_t*>(ko), vout, iout, M, m_dev,
                                      shift - 16, counts, totals, bins, nb2, stream);
}

// ------------------------------------------------------------------ bin edges
// _tile_bin_edges_32bit, splax/_rasterize/_sort/_kernels.py:214-241 (including its M == 1
// behaviour: index 0 writes only the start, so a lone bin stays [0, 0)).

// kKind 2: _tile_bin_edges_64bit (splax/_rasterize/_sort/_kernels.py:244-269), the (image,
// tile) field read from the high word; 0: the packed 32-bit key; 1: the packed key's high half
// (bits 16-31: its image and tile fields, depth_bits >= 16).
constexpr int kKeysPacked = 0, kKeysPackedHigh = 1, kKeysWide = 2;
template <int kKind>
__device__ __forceinline__ int32_t key_bin(const void* keys, int64_t i, int32_t num_tiles,
                                           int32_t tile_bits, int32_t depth_bits) {
    if constexpr (kKind == kKeysWide) {
        const uint64_t k = static_cast<const uint64_t*>(keys)[i] >> 32;
        const uint64_t mask = ((uint64_t)1 << tile_bits) - 1;
        return (int32_t)(k >> tile_bits) * num_tiles + (int32_t)(k & mask);
    } else {
        const int32_t mask = (1 << tile_bits) - 1;
        const int32_t k =
            kKind == kKeysPacked
                ? static_cast<const int32_t*>(keys)[i] >> depth_bits
                : (int32_t)static_cast<const uint16_t*>(keys)[i] >> (depth_bits - 16);
        return (k >> tile_bits) * num_tiles + (k & mask);
    }
}

// Keys per thread of bin_edges_kernel: 8 packed keys, read with one 16-byte load (16-bit key
// halves) or two (32-bit keys) where 4 scalar loads each took more load instructions than the
// kernel's bytes (config 3's bins 18.6 -> 12.2 us); 4 wide keys.
template <int kKind>
constexpr int bin_keys() { return kKind == kKeysWide ? 4 : 8; }

// The tile bin of key word w (kKind's layout).
template <int kKind>
__device__ __forceinline__ int32_t word_bin(uint32_t w, int32_t num_tiles, int32_t tile_bits,
                                            int32_t depth_bits) {
    const int32_t mask = (1 << tile_bits) - 1;
    const int32_t k = kKind == kKeysPacked ? (int32_t)w >> depth_bits
                                           : (int32_t)w >> (depth_bits - 16);
    return (k >> tile_bits) * num_tiles + (k & mask);
}

template <int kKind>
__global__ void __launch_bounds__(256)
bin_edges_kernel(const void* keys, int64_t M_bound, const int32_t* m_dev, int32_t num_tiles,
                 int32_t tile_bits, int32_t depth_bits, int64_t nbins, int32_t* bins) {
    constexpr int KB = bin_keys<kKind>();
    const int64_t M = live_count(m_dev, M_bound);
    // KB consecutive keys and the one before them per thread, all loads issued together
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * KB;
    if (i0 >= M) return;
    int32_t cur[KB];
    if constexpr (kKind == kKeysWide) {
#pragma unroll
        for (int k = 0; k < KB; ++k)
            cur[k] = i0 + k < M ? key_bin<kKind>(keys, i0 + k, num_tiles, tile_bits, depth_bits)
                                : -1;
    } else {
        uint32_t w[KB];
        if (i0 + KB <= M) {
            // whole vectors: i0 is a multiple of 8 keys, so the loads are 16-byte aligned
            if constexpr (kKind == kKeysPackedHigh) {
                const uint4 v = reinterpret_cast<const uint4*>(keys)[i0 / 8];
                const uint32_t p[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    w[2 * k] = p[k] & 0xffffu;
                    w[2 * k + 1] = p[k] >> 16;
                }
            } else {
                const uint4 a = reinterpret_cast<const uint4*>(keys)[i0 / 4];
                const uint4 b = reinterpret_cast<const uint4*>(keys)[i0 / 4 + 1];
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
                w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
            }
#pragma unroll
            for (int k = 0; k < KB; ++k) cur[k] = word_bin<kKind>(w[k], num_tiles, tile_bits, depth_bits);
        } else {
#pragma unroll
            for (int k = 0; k < KB; ++k)
                cur[k] = i0 + k < M ? key_bin<kKind>(keys, i0 + k, num_tiles, tile_bits,
                                                     depth_bits)
                                    : -1;
        }
    }
    const int32_t before =
        i0 > 0 ? key_bin<kKind>(keys, i0 - 1, num_tiles, tile_bits, depth_bits) : -1;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int64_t idx = i0 + k;
        const int32_t c = cur[k];
        // keys emitted from consistent inputs always decode inside [0, nbins)
        if (idx >= M || c < 0 || c >= nbins) continue;
        if (idx == 0) {
            bins[2 * c] = 0;
            continue;
        }
        if (idx == M - 1) bins[2 * c + 1] = (int32_t)M;
        const int32_t prev = k == 0 ? before : cur[k - 1];
        if (prev != c && prev >= 0 && prev < nbins) {
            bins[2 * prev + 1] = (int32_t)idx;
            bins[2 * c] = (int32_t)idx;
        }
    }
}

// ------------------------------------------------------------------ orchestration

// _use_32bit_keys (splax/_rasterize/_sort/_sort.py:23-26), which the reference's tests patch to
// force the 64-bit key; here a process-wide switch (splat_set_wide_keys).
static bool g_force_wide = false;
void set_force_wide_keys(bool force) { g_force_wide = force; }

KeyLayout key_layout(int32_t B, int32_t img_h, int32_t img_w) {
    KeyLayout L;
    L.tiles_x = (img_w + kBlockWidth - 1) / kBlockWidth;
    L.tiles_y = (img_h + kBlockWidth - 1) / kBlockWidth;
    L.num_tiles = L.tiles_x * L.tiles_y;
    auto bit_length = [](int64_t v) {
        int b = 0;
        while (v > 0) {
            ++b;
            v >>= 1;
        }
        return b;
    };
    L.tile_bits = bit_length((int64_t)L.num_tiles - 1);
    L.image_bits = bit_length((int64_t)B - 1);
    L.depth_bits = 31 - L.image_bits - L.tile_bits;
    L.packed = L.depth_bits >= 16 && !g_force_wide;
    L.overflow = !L.packed && L.image_bits + L.tile_bits > 32;
    return L;
}

int run_sort_and_bin(const RasterInputs& in, DeviceScratch& sc, hipStream_t stream,
                     int64_t* M_out, KeyLayout* lay_out, const SortTargets* tgt,
                     SortOutputs* out, bool full_keys) {
    const int32_t B = in.B_geom;
    const KeyLayout L = key_layout(B, in.img_h, in.img_w);
    *lay_out = L;
    if (L.overflow) {
        return fail(kErrKeyOverflow,
                    "batched intersection key overflow: image_n_bits(" +
                        std::to_string(L.image_bits) + ") + tile_n_bits(" +
                        std::to_string(L.tile_bits) + ") = " +
                        std::to_string(L.image_bits + L.tile_bits) + " > 32 (batch B=" +
                        std::to_string(B) + ", n_tiles=" + std::to_string(L.num_tiles) +
                        "). Reduce batch size or resolution.");
    }
    const bool wide = !L.packed;
    // the sort's digits: four bytes of the (quantized or raw float) depth, then for the 64-bit
    // key the bytes of the (image, tile) field above bit 32
    PassShifts ps;
    ps.n = 0;
    for (int b = 0; b < 4; ++b) ps.shift[ps.n++] = 8 * b;
    if (wide)
        for (int b = 0; b < (L.image_bits + L.tile_bits + 7) / 8; ++b) ps.shift[ps.n++] = 32 + 8 * b;
    const int last_dst = ((ps.n - 1) & 1) ? 0 : 1;  // buffer the last pass writes
    // packed keys whose sorted form nobody reads end as their 16-bit high halves
    const bool narrow = !wide && !full_keys;
    // a kept forward given no position buffer (no backward will read its lists) sorts no
    // emission positions
    const bool with_pos = !(tgt && tgt->ids && !tgt->pos);
    const int64_t total = (int64_t)B * in.n;
    const int64_t nbins = (int64_t)B * L.num_tiles;
    int rc = sc.ensure_sort(0, nbins, B, wide);
    if (rc) return rc;
    int32_t* bins = (tgt && tgt->bins) ? tgt->bins : sc.tile_bins;
    SortOutputs o;
    o.bins = bins;
    o.wide = wide;
    o.high_keys = narrow;
    if (out) *out = o;
    const bool known = tgt && tgt->M_known >= 0;
    if (total <= 0) {
        *M_out = 0;
        return fill_zero_i32(bins, 2 * nbins, stream);
    }
    // The one device-to-host read: the intersection count (skipped when the caller supplies it).
    // The copy is enqueued first (on the render path the chunk scan has already stored the count
    // into the pinned word, so only the event is recorded); the depth range launches run while
    // the host waits
    // (splax/_rasterize/_sort/_sort.py:71-96). With a capacity-bounded target the host does not
    // wait here at all: every launch below is sized by the capacity and bounded on the device by
    // the count itself (live_count), and the caller settles the count after its last launch
    // (settle_count), so the host never stalls the stream between the projection and the blend.
    const bool deferred = !known && tgt && tgt->capacity >= 0;
    const int32_t* count_src = tgt && tgt->count_src ? tgt->count_src : in.cum + (total - 1);
    const bool on_host = tgt && tgt->count_on_host;  // already stored by its kernel
    if (!known && ((!on_host && hipMemcpyAsync(sc.pinned_count, count_src, sizeof(int32_t),
                                               hipMemcpyDeviceToHost, stream) != hipSuccess) ||
                   hipEventRecord(sc.count_event, stream) != hipSuccess))
        return fail(kErrRuntime, "count readback enqueue failed");
    const float* depth_mm = sc.depth_mm;
    if (!wide && tgt && tgt->depth_mm) {
        depth_mm = tgt->depth_mm;  // formed by the fused projection
    } else if (!wide) {  // the 64-bit key carries the raw depth: no depth range
        const int32_t bpi =
            (int32_t)((in.n + kMmThreads * kMmItems - 1) / (kMmThreads * kMmItems));
        if ((int64_t)bpi * B * 2 > sc.mm_partial_cap)
            return fail(kErrRuntime, "depth-range partials not allocated");
        StageTimer tm(stream, kStageMinmax);
        hipLaunchKernelGGL(minmax_partial_kernel, dim3(bpi, B), dim3(kMmThreads), 0, stream,
                           in.depths, in.radii, in.n, bpi, sc.mm_partial);
        hipLaunchKernelGGL(minmax_final_kernel, dim3(B), dim3(kMmThreads), 0, stream,
                           sc.mm_partial, bpi, sc.depth_mm);
        if (hipGetLastError() != hipSuccess) return fail(kErrLaunch, "minmax launch failed");
    }
    // M: the count, or with a deferred count its bound (the capacity); m_dev then points at the
    // count in device memory and m_est (the previous settled count, for the partition shape
    // only) stands in for it on the host
    int64_t M;
    const int32_t* m_dev = nullptr;
    if (known) {
        M = tgt->M_known;
    } else if (deferred) {
        M = tgt->capacity;
        m_dev = count_src;
    } else {
        if (hipEventSynchronize(sc.count_event) != hipSuccess)
            return fail(kErrRuntime, "count readback failed");
        M = *sc.pinned_count;
    }
    if (!deferred) {
        if (M < 0) return fail(kErrTooMany, "intersection count overflowed int32");
        if (M >= ((int64_t)1 << 31)) return fail(kErrTooMany, "more than 2^31 - 1 intersections");
        if (tgt && tgt->capacity >= 0 && M > tgt->capacity)
            return fail(kErrTooMany, "sorted-list buffers hold " + std::to_string(tgt->capacity) +
                                         " intersections, " + std::to_string(M) + " needed");
    }
    *M_out = deferred ? -1 : M;
    o.count_deferred = deferred;
    if (out) *out = o;
    const int64_t m_est =
        deferred && sc.last_count >= 0 && sc.last_count < M ? sc.last_count : M;
    rc = sc.ensure_sort(M, nbins, B, wide);
    if (rc) return rc;
    const uint32_t* chunk_prefix = tgt ? tgt->chunk_prefix : nullptr;
    if (M == 0) {
        // no emission: the chunk-local cum_tiles_hit is finalized here
        if (chunk_prefix) {
            rc = launch_chunk_offsets(const_cast<int32_t*>(in.cum), total, chunk_prefix, stream);
            if (rc) return fail(rc, "chunk offset launch failed");
        }
        return fill_zero_i32(bins, 2 * nbins, stream);
    }
    int32_t* ids_final = (tgt && tgt->ids) ? tgt->ids : sc.gids[last_dst];
    int32_t* pos_final = (tgt && tgt->pos) ? tgt->pos : sc.vals[last_dst];
    void* kbuf[2] = {wide ? (void*)sc.wkeys[0] : (void*)sc.keys[0],
                     wide ? (void*)sc.wkeys[1] : (void*)sc.keys[1]};
    o.keys = kbuf[last_dst];
    o.ids = ids_final;
    o.pos = with_pos ? pos_final : nullptr;
    if (out) *out = o;

    {
        StageTimer tm(stream, kStageEmit);
        EmitParams E;
        E.xys = in.xys; E.depths = in.depths; E.radii = in.radii; E.conics = in.conics;
        E.map_opac = in.map_opac; E.rows_map_opac = in.rows_map_opac;
        E.cum = in.cum; E.mm = depth_mm; E.n = in.n; E.total = total; E.M = M; E.m_dev = m_dev;
        E.chunk_prefix = chunk_prefix;
        E.nth = tgt ? tgt->num_tiles_hit : nullptr;
        E.cum_fix = const_cast<int32_t*>(in.cum);
        E.tiles_x = L.tiles_x; E.tiles_y = L.tiles_y; E.tile_bits = L.tile_bits;
        E.depth_bits = L.depth_bits; E.keys = kbuf[0]; E.owner = sc.gids[0];
        const dim3 grid((unsigned)((total + 255) / 256));
        if (wide)
            hipLaunchKernelGGL(emit_keys_kernel<true>, grid, dim3(256), 0, stream, E);
        else
            hipLaunchKernelGGL(emit_keys_kernel<false>, grid, dim3(256), 0, stream, E);
        if (hipGetLastError() != hipSuccess) return fail(kErrLaunch, "emit launch failed");
    }
    {
        StageTimer tm(stream, kStageSort);
        // 64-bit keys: 8192-key partitions from 1M keys on (digit runs of about 32 keys leave as
        // whole 128-byte lines), 4096-key partitions below, so small sorts still spread over the
        // CUs
        const bool big = m_est >= kSortBigM;
        // packed keys: one partition per workgroup and two 1024-thread workgroups per CU. The
        // smallest of 4..8 keys per thread whose partitions all fit in one round of workgroups,
        // else 8: a second round that only a few partitions occupy costs nearly a whole round
        // (at 2.66M keys, 6 keys per thread sort in 0.109 ms, 5 in 0.128 and 8 in 0.121)
        const int64_t slots = 2 * (int64_t)(sc.compute_units > 0 ? sc.compute_units : 256);
        int items = 8;
        for (int k = 4; k < 8; ++k) {
            if ((m_est + (int64_t)k * kSortThreads - 1) / ((int64_t)k * kSortThreads) <= slots) {
                items = k;
                break;
            }
        }
        // passes ping-pong 0 -> 1 -> 0 ...; the first pass generates the emission positions,
        // the last writes positions and items straight into their final buffers (the caller's
        // when it keeps the sorted lists)
        for (int pass = 0; pass < ps.n; ++pass) {
            const int src = pass & 1, dst = 1 - src;
            const bool last = pass == ps.n - 1;
            const int32_t* vin = pass == 0 || !with_pos ? nullptr : sc.vals[src];
            int32_t* vout = !with_pos ? nullptr : last ? pos_final : sc.vals[dst];
            int32_t* iout = last ? ids_final : sc.gids[dst];
            const int shift = ps.shift[pass];
            const int64_t nb2 = pass == 0 ? 2 * nbins : 0;
            if (wide) {
                const uint64_t* ki = sc.wkeys[src];
                uint64_t* ko = sc.wkeys[dst];
                if (big)
                    launch_pass<uint64_t, 8>(ki, vin, sc.gids[src], ko, vout, iout, M, m_dev, shift,
                                             sc.part_counts, sc.hist, bins, nb2, stream);
                else
                    launch_pass<uint64_t, 4>(ki, vin, sc.gids[src], ko, vout, iout, M, m_dev, shift,
                                             sc.part_counts, sc.hist, bins, nb2, stream);
            } else {
                // narrow: the pass over bits 8-15 writes the keys' high halves and the passes
                // over bits 16-30 move 16-bit keys (the buffers hold either)
                const int kind = !narrow || pass == 0 ? 0 : pass == 1 ? 1 : 2;
                const void* ki = sc.keys[src];
                void* ko = sc.keys[dst];
                const int32_t* gi = sc.gids[src];
                uint32_t* pc = sc.part_counts;
                switch (items) {
                case 4:
                    packed_pass<4>(kind, ki, vin, gi, ko, vout, iout, M, m_dev, shift, pc,
                                   sc.hist, bins, nb2, stream);
                    break;
                case 5:
                    packed_pass<5>(kind, ki, vin, gi, ko, vout, iout, M, m_dev, shift, pc,
                                   sc.hist, bins, nb2, stream);
                    break;
                case 6:
                    packed_pass<6>(kind, ki, vin, gi, ko, vout, iout, M, m_dev, shift, pc,
                                   sc.hist, bins, nb2, stream);
                    break;
                case 7:
                    packed_pass<7>(kind, ki, vin, gi, ko, vout, iout, M, m_dev, shift, pc,
                                   sc.hist, bins, nb2, stream);
                    break;
                default:
                    packed_pass<8>(kind, ki, vin, gi, ko, vout, iout, M, m_dev, shift, pc,
                                   sc.hist, bins, nb2, stream);
                }
            }
        }
        if (hipGetLastError() != hipSuccess) return fail(kErrLaunch, "sort launch failed");
    }
    {
        StageTimer tm(stream, kStageBins);
        const int kb = wide ? bin_keys<kKeysWide>() : bin_keys<kKeysPacked>();
        const dim3 grid((unsigned)((M + 256 * kb - 1) / (256 * kb)));
        if (wide)
            hipLaunchKernelGGL(bin_edges_kernel<kKeysWide>, grid, dim3(256), 0, stream, o.keys,
                               M, m_dev, L.num_tiles, L.tile_bits, L.depth_bits, nbins, bins);
        else if (narrow)
            hipLaunchKernelGGL(bin_edges_kernel<kKeysPackedHigh>, grid, dim3(256), 0, stream,
                               o.keys, M, m_dev, L.num_tiles, L.tile_bits, L.depth_bits, nbins,
                               bins);
        else
            hipLaunchKernelGGL(bin_edges_kernel<kKeysPacked>, grid, dim3(256), 0, stream,
                               o.keys, M, m_dev, L.num_tiles, L.tile_bits, L.depth_bits, nbins,
                               bins);
        if (hipGetLastError() != hipSuccess) return fail(kErrLaunch, "bins launch failed");
    }
    return 0;
}

int settle_count(DeviceScratch& sc, int64_t capacity, int64_t* M_out) {
    if (hipEventSynchronize(sc.count_event) != hipSuccess)
        return fail(kErrRuntime, "count readback failed");
    const int64_t M = *sc.pinned_count;
    *M_out = M;
    if (M < 0) return fail(kErrTooMany, "intersection count overflowed int32");
    sc.last_count = M;
    if (M > capacity)
        return fail(kErrTooMany, "sorted-list buffers hold " + std::to_string(capacity) +
                                     " intersections, " + std::to_string(M) + " needed");
    return 0;
}

}  // namespace splat
