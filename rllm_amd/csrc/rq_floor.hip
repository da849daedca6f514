// Read floor of a dot4 matvec launch, the reference point of bench.py's
// roofline (built into its own librq_floor.so; librq.so does not contain it).
//
// rq_floor_read reads a buffer laid out as a tiled weight's chunk plane
// (rq_params.h): `tiles` tiles of C chunks, each chunk 64 lanes x 16 B, one
// wave per tile, four waves per 256-thread workgroup, every load a 16-byte
// nontemporal load contiguous across the wave: the bytes, launch shape and
// load pattern of rq_mvx_<fmt>_1 over such a weight. Instead of the matvec's
// activation staging, dot products and scaling it folds the loaded words
// with XOR, reduces them over each row's lane group with the same DPP steps
// and stores one 4-byte word per row, as the matvec stores one f32 per row.
// Its time is what a launch of that shape costs for its memory traffic alone.
// rq_floor_empty launches the same grid with no work at all: the fixed cost
// of one dependent launch in a replayed graph.

#include <string.h>

#include "rq_device.h"

template <int C>
__global__ __launch_bounds__(256) void rq_floor_read_k(const u8* __restrict__ base, int64_t tiles, int g,
                                                        u32* __restrict__ out, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tiles) return;  // wave-uniform
    const u8* p = base + (t * C * 64 + lane) * 16;
    int4 v[C];
#pragma unroll
    for (int c = 0; c < C; c++) v[c] = ld16_nt(p + c * 1024);
    int x = 0;
#pragma unroll
    for (int c = 0; c < C; c++) x ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
    // The row's lanes meet (g = 64 / rows per tile lanes, a power of two <= 16).
    if (g >= 2) x ^= dpp_i<DPP_QUAD_1032>(x);
    if (g >= 4) x ^= dpp_i<DPP_QUAD_2301>(x);
    if (g >= 8) x ^= dpp_i<DPP_ROW_HALF_MIRROR>(x);
    if (g >= 16) x ^= dpp_i<DPP_ROW_MIRROR>(x);
    const int64_t row = t * (64 / g) + lane / g;
    if ((lane & (g - 1)) == 0 && row < rows) out[row] = (u32)x;
}

// Launches the read floor on `stream` over tiles x chunks x 1 KiB at `base`
// (16-byte aligned) for tiles of 64 / lanes_per_row rows; out holds `rows`
// words. chunks: 9 (Q4_K, Q4_0), 13 (Q6_K) or 17 (Q8_0). Returns a hipError_t.
extern "C" int rq_floor_read(const void* base, int64_t tiles, int chunks, int lanes_per_row, void* out, int64_t rows,
                             void* stream) {
    if (!base || !out || tiles <= 0 || rows <= 0 || lanes_per_row < 1 || lanes_per_row > 16 ||
        (lanes_per_row & (lanes_per_row - 1)) != 0 || rows > tiles * (64 / lanes_per_row) ||
        ((uintptr_t)base & 15) != 0)
        return (int)hipErrorInvalidValue;
    const dim3 grid((unsigned)((tiles + 3) / 4)), block(256);
    hipStream_t s = (hipStream_t)stream;
    const u8* b = (const u8*)base;
    switch (chunks) {
    case 9: hipLaunchKernelGGL(rq_floor_read_k<9>, grid, block, 0, s, b, tiles, lanes_per_row, (u32*)out, rows); break;
    case 13: hipLaunchKernelGGL(rq_floor_read_k<13>, grid, block, 0, s, b, tiles, lanes_per_row, (u32*)out, rows); break;
    case 17: hipLaunchKernelGGL(rq_floor_read_k<17>, grid, block, 0, s, b, tiles, lanes_per_row, (u32*)out, rows); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// The general form, for every launch of the decode step: up to three
// targets (the mixed q/k/v launch), tiles of R rows x S super-blocks as the
// dot4 layout stores them (R = 1 for rows of more than 32 super-blocks, as
// ffn_down's 56), the Q6_K scale plane (2 B per slot), and `pair` = 1 for
// the gated FFN's workgroups, whose wave w reads tile w of both gate and up.
// Lane to slot mapping, padding lanes and the row reduction are the matvec's
// (tile_lane, group_sum); the reads are its loads, with no arithmetic.
struct RqFloorTarget {
    const u8* base;  // chunk plane
    const u8* tail;  // Q6_K f16 d per slot, or null
    int64_t tiles;
    int32_t chunks, R, S, pad;
    u32* out;        // one word per row
    int64_t rows;
    int64_t wave0;   // first wave of the target (pair: 0 for both)
};
struct RqFloorParams {
    int32_t count;  // first: loaded in the same batch as the targets
    int32_t pair;
    RqFloorTarget t[3];
};

// One tile's loads (C chunks, unrolled and unguarded as the matvec issues
// them, then the scale-plane word), folded with XOR.
template <int C>
__device__ __forceinline__ int floor_tile_c(const RqFloorTarget& T, int64_t tile, int lane, int& row) {
    // The matvec's tile_lane: rows of 64 / R lanes (R = 1: the whole wave).
    const int sh = 6 - __builtin_ctz(T.R);
    row = lane >> sh;
    const int col = lane & ((1 << sh) - 1);
    const bool real = col < T.S;
    const int64_t slots = (int64_t)T.R * T.S;
    const int64_t slot = row * T.S + (real ? col : 0);
    const u8* p = T.base + (tile * C * slots + slot) * 16;
    int4 v[C];
#pragma unroll
    for (int c = 0; c < C; c++) v[c] = ld16_nt(p + c * slots * 16);
    int x = T.tail ? (int)*gmem((const u16*)(T.tail + (tile * slots + slot) * 2)) : 0;
#pragma unroll
    for (int c = 0; c < C; c++) x ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
    return x;
}

// C = 0: the target's chunk count picks the path (wave-uniform; the mixed
// q/k/v launch); otherwise every target has C chunks, which keeps the
// registers (and the occupancy) those of one format.
template <int C>
__device__ __forceinline__ int floor_tile(const RqFloorTarget& T, int64_t tile, int lane, int& row) {
    if (C != 0) return floor_tile_c<C == 0 ? 9 : C>(T, tile, lane, row);
    if (T.chunks == 9) return floor_tile_c<9>(T, tile, lane, row);
    return floor_tile_c<13>(T, tile, lane, row);
}

__device__ __forceinline__ void floor_store(const RqFloorTarget& T, int64_t tile, int lane, int row, int x) {
    const int g = T.R > 1 ? 64 >> __builtin_ctz(T.R) : 64;
    if (g >= 2) x ^= dpp_i<DPP_QUAD_1032>(x);
    if (g >= 4) x ^= dpp_i<DPP_QUAD_2301>(x);
    if (g >= 8) x ^= dpp_i<DPP_ROW_HALF_MIRROR>(x);
    if (g >= 16) x ^= dpp_i<DPP_ROW_MIRROR>(x);
    if (g == 32) x ^= dpp_i<DPP_ROW_BCAST15, 0xA>(x);
    if (g == 64)
        x = (__builtin_amdgcn_readlane(x, 0) ^ __builtin_amdgcn_readlane(x, 16)) ^
            (__builtin_amdgcn_readlane(x, 32) ^ __builtin_amdgcn_readlane(x, 48));
    const bool leader = g == 32 ? (lane & 31) == 16 : (g == 64 ? lane == 0 : (lane & (g - 1)) == 0);
    const int64_t r = tile * T.R + row;
    if (leader && row < T.R && r < T.rows) gmem(T.out)[r] = (u32)x;
}

// Every target's fields in one batch of kernarg loads (the matvec kernels'
// pick_target): a reference indexed by the runtime target number would
// reload its fields with dependent kernarg loads ahead of the first weight
// load. floor_pick then takes the wave's target by value; a one-target
// launch takes the first with no selects.
__device__ __forceinline__ void floor_load(const RqFloorParams& P, RqFloorTarget& a, RqFloorTarget& b,
                                           RqFloorTarget& c) {
#define RQ_FLOAD(f)               \
    a.f = sgpr_value(P.t[0].f); \
    b.f = sgpr_value(P.t[1].f); \
    c.f = sgpr_value(P.t[2].f);
    RQ_FLOAD(base) RQ_FLOAD(tail) RQ_FLOAD(tiles) RQ_FLOAD(chunks) RQ_FLOAD(R) RQ_FLOAD(S) RQ_FLOAD(out)
    RQ_FLOAD(rows) RQ_FLOAD(wave0)
#undef RQ_FLOAD
    a.pad = b.pad = c.pad = 0;
}

__device__ __forceinline__ RqFloorTarget floor_pick(const RqFloorParams& P, int64_t gw) {
    RqFloorTarget a, b, c;
    const int count = sgpr_value(P.count);
    floor_load(P, a, b, c);
    if (count == 1) return a;
    const int ti = (int)(gw >= b.wave0) + (int)(gw >= c.wave0 && count > 2);
    RqFloorTarget r;
#define RQ_FPICK(f) r.f = ti == 0 ? a.f : (ti == 1 ? b.f : c.f);
    RQ_FPICK(base) RQ_FPICK(tail) RQ_FPICK(tiles) RQ_FPICK(chunks) RQ_FPICK(R) RQ_FPICK(S) RQ_FPICK(out)
    RQ_FPICK(rows) RQ_FPICK(wave0)
#undef RQ_FPICK
    r.pad = 0;
    return r;
}

template <int THREADS, bool PAIR, int C>
__global__ __launch_bounds__(THREADS) void rq_floor_many_k(RqFloorParams P) {
    const int lane = threadIdx.x & 63;
    // Wave-uniform (readfirstlane): the target pick and tile index stay scalar.
    const int64_t gw = (int64_t)blockIdx.x * (THREADS / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (PAIR) {
        RqFloorTarget A, B, unused;
        floor_load(P, A, B, unused);
        if (gw >= A.tiles) return;  // wave-uniform
        int r0, r1;
        const int x0 = floor_tile<C>(A, gw, lane, r0);
        const int x1 = floor_tile<C>(B, gw, lane, r1);
        floor_store(A, gw, lane, r0, x0);
        floor_store(B, gw, lane, r1, x1);
        return;
    }
    const RqFloorTarget T = floor_pick(P, gw);
    const int64_t tile = gw - T.wave0;
    if (tile >= T.tiles) return;  // wave-uniform
    int row;
    const int x = floor_tile<C>(T, tile, lane, row);
    floor_store(T, tile, lane, row, x);
}

// Launches the general read floor: `count` targets one after the other in
// the grid (or, with pair, two targets of equal tile counts side by side in
// each wave, 512 threads), `threads` per workgroup (256 or 1024). Targets of
// different chunk counts only as Q4_K + Q6_K at 256 threads. Returns a
// hipError_t.
extern "C" int rq_floor_read_many(const void* targets, int count, int pair, int threads, void* stream) {
    if (!targets || count < 1 || count > 3 || (pair && (count != 2 || threads != 512)) ||
        (!pair && threads != 256 && threads != 1024))
        return (int)hipErrorInvalidValue;
    RqFloorParams P;
    memset(&P, 0, sizeof P);
    memcpy(P.t, targets, sizeof(RqFloorTarget) * count);
    int64_t waves = 0;
    int c0 = ((const RqFloorTarget*)targets)[0].chunks;
    bool same = true;
    for (int i = 0; i < count; i++) {
        RqFloorTarget& T = P.t[i];
        if (!T.base || !T.out || T.tiles <= 0 || T.rows <= 0 || T.R < 1 || T.R > 64 || (T.R & (T.R - 1)) ||
            T.S < 1 || T.S > 64 || (T.R > 1 && T.S > 64 / T.R) || T.rows > T.tiles * T.R ||
            (T.chunks != 9 && T.chunks != 13 && T.chunks != 17) || ((uintptr_t)T.base & 15))
            return (int)hipErrorInvalidValue;
        same = same && T.chunks == c0;
        T.wave0 = pair ? 0 : waves;
        waves = pair ? T.tiles : waves + T.tiles;
    }
    if (pair && P.t[0].tiles != P.t[1].tiles) return (int)hipErrorInvalidValue;
    P.count = count;
    P.pair = pair;
    const int wpg = threads / 64;
    const dim3 grid((unsigned)((waves + wpg - 1) / wpg)), block(threads);
    hipStream_t s = (hipStream_t)stream;
    // Launch shapes of the decode step: one format per launch (9, 13 or 17
    // chunks) at 256 or 1024 threads, the mixed Q4_K / Q6_K one at 256, the
    // gated FFN's pairs (Q4_K, Q4_0: 9; Q6_K: 13) at 512.
    if (!same && (c0 + ((const RqFloorTarget*)targets)[count - 1].chunks != 22 || threads != 256 || pair))
        return (int)hipErrorInvalidValue;
#define RQ_FLOOR_LAUNCH(TH, PR, CC) hipLaunchKernelGGL((rq_floor_many_k<TH, PR, CC>), grid, block, 0, s, P)
    if (!same)
        RQ_FLOOR_LAUNCH(256, false, 0);
    else if (pair && c0 == 9)
        RQ_FLOOR_LAUNCH(512, true, 9);
    else if (pair && c0 == 13)
        RQ_FLOOR_LAUNCH(512, true, 13);
    else if (pair)
        return (int)hipErrorInvalidValue;
    else if (threads == 256 && c0 == 9)
        RQ_FLOOR_LAUNCH(256, false, 9);
    else if (threads == 256 && c0 == 13)
        RQ_FLOOR_LAUNCH(256, false, 13);
    else if (threads == 256)
        RQ_FLOOR_LAUNCH(256, false, 17);
    else if (threads == 1024 && c0 == 9)
        RQ_FLOOR_LAUNCH(1024, false, 9);
    else if (threads == 1024 && c0 == 13)
        RQ_FLOOR_LAUNCH(1024, false, 13);
    else if (threads == 1024)
        RQ_FLOOR_LAUNCH(1024, false, 17);
    else
        return (int)hipErrorInvalidValue;
#undef RQ_FLOOR_LAUNCH
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Other launch shapes of the same read (rq_floor_read's tiles of C = 9
// chunks, 16-byte nontemporal loads contiguous across a wave, XOR fold, one
// word per 16 lanes): does any shape read the bytes faster?
//   kind 1: one tile per wave, `threads` per workgroup;
//   kind 2: two consecutive tiles per wave, all 18 loads issued first;
//   kind 3: grid-stride, wave w reads tiles w, w + W, ... (W waves in all);
//   kind 4: kind 1 with each XCD's workgroups on one contiguous eighth.
template <int TPW, bool XCD = false>
__global__ __launch_bounds__(1024) void rq_floor_shape_k(const u8* __restrict__ base, int64_t tiles,
                                                         u32* __restrict__ out) {
    constexpr int C = 9;
    const int lane = threadIdx.x & 63;
    // XCD: workgroup b runs on XCD b % 8 (round-robin dispatch); it takes
    // workgroup slot (b % 8) * (G / 8) + b / 8, so that each XCD reads one
    // contiguous eighth of the buffer (G a multiple of 8).
    const int64_t bx = XCD ? (int64_t)(blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int64_t w = bx * (blockDim.x >> 6) + (threadIdx.x >> 6);
    int4 v[TPW][C];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int64_t t = w * TPW + j;
#pragma unroll
        for (int c = 0; c < C; c++) v[j][c] = t < tiles ? ld16_nt(base + ((t * C + c) * 64 + lane) * 16) : make_int4(0, 0, 0, 0);
    }
    int x = 0;
#pragma unroll
    for (int j = 0; j < TPW; j++)
#pragma unroll
        for (int c = 0; c < C; c++) x ^= v[j][c].x ^ v[j][c].y ^ v[j][c].z ^ v[j][c].w;
    x ^= dpp_i<DPP_QUAD_1032>(x);
    x ^= dpp_i<DPP_QUAD_2301>(x);
    x ^= dpp_i<DPP_ROW_HALF_MIRROR>(x);
    x ^= dpp_i<DPP_ROW_MIRROR>(x);
    if (w * TPW < tiles && (lane & 15) == 0) out[w * 4 + (lane >> 4)] = (u32)x;
}

__global__ __launch_bounds__(1024) void rq_floor_stride_k(const u8* __restrict__ base, int64_t tiles,
                                                          u32* __restrict__ out) {
    constexpr int C = 9;
    const int lane = threadIdx.x & 63;
    const int64_t W = (int64_t)gridDim.x * (blockDim.x >> 6);
    const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    int x = 0;
    for (int64_t t = w; t < tiles; t += W) {
        int4 v[C];
#pragma unroll
        for (int c = 0; c < C; c++) v[c] = ld16_nt(base + ((t * C + c) * 64 + lane) * 16);
#pragma unroll
        for (int c = 0; c < C; c++) x ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
    }
    x ^= dpp_i<DPP_QUAD_1032>(x);
    x ^= dpp_i<DPP_QUAD_2301>(x);
    x ^= dpp_i<DPP_ROW_HALF_MIRROR>(x);
    x ^= dpp_i<DPP_ROW_MIRROR>(x);
    if (w < tiles && (lane & 15) == 0) out[w * 4 + (lane >> 4)] = (u32)x;
}

// Launches shape `kind` over `tiles` tiles of 9 KiB at `base` (16-byte
// aligned) in `grid` workgroups of `threads` (64 .. 1024, a multiple of 64);
// out holds 4 x tiles words. Kinds 1 and 2 need grid x threads / 64 x kind
// >= tiles. Returns a hipError_t.
extern "C" int rq_floor_shape(int kind, const void* base, int64_t tiles, int threads, int64_t grid, void* out,
                              void* stream) {
    if (!base || !out || tiles <= 0 || threads < 64 || threads > 1024 || threads % 64 != 0 || grid <= 0 ||
        grid > 0x7fffffff || ((uintptr_t)base & 15) != 0)
        return (int)hipErrorInvalidValue;
    const int64_t waves = grid * (threads / 64);
    if ((kind == 1 || kind == 2 || kind == 4) && waves * (kind == 2 ? 2 : 1) < tiles) return (int)hipErrorInvalidValue;
    if (kind == 4 && grid % 8 != 0) return (int)hipErrorInvalidValue;
    hipStream_t s = (hipStream_t)stream;
    const u8* b = (const u8*)base;
    switch (kind) {
    case 1: hipLaunchKernelGGL(rq_floor_shape_k<1>, dim3((unsigned)grid), dim3(threads), 0, s, b, tiles, (u32*)out); break;
    case 2: hipLaunchKernelGGL(rq_floor_shape_k<2>, dim3((unsigned)grid), dim3(threads), 0, s, b, tiles, (u32*)out); break;
    case 3: hipLaunchKernelGGL(rq_floor_stride_k, dim3((unsigned)grid), dim3(threads), 0, s, b, tiles, (u32*)out); break;
    case 4: hipLaunchKernelGGL((rq_floor_shape_k<1, true>), dim3((unsigned)grid), dim3(threads), 0, s, b, tiles, (u32*)out); break;
    default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

__global__ __launch_bounds__(256) void rq_floor_empty_k() {}

// Launches `workgroups` empty 256-thread workgroups on `stream`. Returns a
// hipError_t.
extern "C" int rq_floor_empty(int64_t workgroups, void* stream) {
    if (workgroups <= 0 || workgroups > 0x7fffffff) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(rq_floor_empty_k, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

// A kernel of known duration, which converts clock-cycle counters (rocprofv3
// --pmc GRBM_GUI_ACTIVE) of other kernels to time: every wave reads the
// 100 MHz real-time counter at its start and loops until it has advanced by
// `ticks`, so the launch lasts `ticks` x 10 ns plus its ramp; two lengths
// give the counter's cycles per microsecond as their difference. The wait
// ends for every wave (the counter is free-running); no memory is written.
__global__ __launch_bounds__(64) void rq_floor_spin_k(uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    uint64_t t = t0;
    while (t - t0 < ticks) t = __builtin_amdgcn_s_memrealtime();
}

// Launches `workgroups` one-wave workgroups of rq_floor_spin_k that each run
// `ticks` (1 .. 10^6, at most 10 ms) of the real-time counter. Returns a
// hipError_t.
extern "C" int rq_floor_spin(uint64_t ticks, int64_t workgroups, void* stream) {
    if (ticks < 1 || ticks > 1000000 || workgroups <= 0 || workgroups > 65536) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(rq_floor_spin_k, dim3((unsigned)workgroups), dim3(64), 0, (hipStream_t)stream, ticks);
    return (int)hipGetLastError();
}
