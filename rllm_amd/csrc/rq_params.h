// Kernel parameter blocks shared by the host library (rq_host.cpp, g++) and
// the gfx950 kernels (rq_kernels.hip, hipcc). Plain-old-data only, passed by
// value as the single kernel argument.
//
// Device weight layout ("RQ layout"). A weight of n rows and k columns has
// U = k/32 units (32 consecutive elements of a row) per row and SB = k/256
// super-blocks for the K-quants. It lives in up to four planes, each a
// row-major array with its own row stride in bytes:
//
//   Q4_0  p0: 16 B per unit, byte b = q[b] | q[b+16] << 4 (GGUF's own order)
//         p1: f16 d per unit
//   Q8_0  p0: int8 codes, a row = [bytes 0..15 of every unit][bytes 16..31 of
//             every unit], so each lane's two 16-byte loads are both
//             contiguous across the wave
//         p1: f16 d per unit
//   Q4_K  p0: 16 B per unit (sub-block), byte b = q[b] | q[b+16] << 4
//         p1: 16 B per super-block, GGUF's d, dmin and packed 6-bit
//             scales/mins verbatim (unpacked in registers)
//   Q6_K  p0: 16 B per unit, low nibbles, byte b = lo(q[b]) | lo(q[b+16]) << 4
//         p1: 8 B per unit, high 2-bit pairs: dword h (elements 16h..16h+15)
//             holds element 16h+4c+i's bits at bit 8i + 2c (c, i < 4)
//         p2: the unit's two int8 sub-scales (elements 0-15, 16-31)
//         p3: f16 d per super-block
//
// Every format keeps GGUF's byte count (18/34/144/210 bytes per block): the
// repack only moves bytes, it adds none and rounds nothing.
#pragma once

#include <stdint.h>

#define RQ_FMT_Q4_0 0
#define RQ_FMT_Q8_0 1
#define RQ_FMT_Q4_K 2
#define RQ_FMT_Q6_K 3
#define RQ_NUM_FMTS 4

// Threads per matvec workgroup (4 waves of 64).
#define RQ_MV_THREADS 256
#define RQ_MV_WAVES (RQ_MV_THREADS / 64)
// Weights sharing one activation in one launch (Q/K/V, gate/up).
#define RQ_MV_TARGETS 3
// Most activation columns per matvec launch.
#define RQ_MV_MAX_NC 8

// Rows each wave streams, by activation column count (compile-time in the
// kernels, mirrored here for the host's grid sizing).
static inline int rq_mv_rows_per_wave(int nc) { return nc <= 2 ? 4 : (nc <= 4 ? 2 : 1); }

struct RqPlanes {
    const uint8_t* p[4];
    int64_t stride[4];
};

struct RqMvTarget {
    RqPlanes w;
    float* out;       // out[j * n + r]
    int32_t n;        // rows
    int32_t wave_start;  // first global wave index of this target
};

struct RqMvParams {
    RqMvTarget t[RQ_MV_TARGETS];
    const int8_t* xq;    // Q8_1 codes, column j at xq + j * k
    const uint16_t* xd;  // Q8_1 f16 scales, column j at xd + j * k / 32
    int32_t count;
    int32_t k;
    int32_t m;  // columns in this launch (<= the kernel's NC)
    int32_t pad;
};

struct RqQuantParams {
    const float* x;
    int8_t* qs;
    uint16_t* d;
    uint16_t* s;
    int64_t nblocks;  // m * k / 32
};

struct RqRepackParams {
    const uint8_t* raw;  // GGUF bytes of rows [row0, row0 + rows)
    uint8_t* p[4];
    int64_t stride[4];
    int64_t row0;
    int64_t rows;
    int32_t k;
    int32_t pad;
};

struct RqDotsParams {
    RqPlanes w;
    const int8_t* xq;
    const uint16_t* xd;
    int32_t* dots;
    int64_t n;
    int32_t k;
    int32_t m;
};
