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

__global__ __launch_bounds__(256) void rq_floor_empty_k() {}

// Launches `workgroups` empty 256-thread workgroups on `stream`. Returns a
// hipError_t.
extern "C" int rq_floor_empty(int64_t workgroups, void* stream) {
    if (workgroups <= 0 || workgroups > 0x7fffffff) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(rq_floor_empty_k, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}
