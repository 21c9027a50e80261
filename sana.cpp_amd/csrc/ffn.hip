// K5: Mix-FFN depthwise 3x3 conv + GLU gate, fused, on a token-major grid.
//
// Replaces, in glumb_conv (src/common_ops.cpp:733-761): depthwise_conv2d_3x3
// (zero padding, taps summed in (ky, kx) order, then + bias; :483-505),
// split_channels_4d (src/tensor.cpp:465-493), SiLU of the gate half and the
// data * gate product.  The SiLU after the inverted 1x1 conv is fused into the
// producing GEMM's epilogue, so the input here is already silu(inv(x) + b).
//
// Layout: channels are contiguous per token, so 8 channels of one token are
// one 16-byte load and consecutive lanes read consecutive 16-byte channel
// groups of the same token (coalesced).  Depthwise weights are stored
// tap-major [9][E] so the 8 weights of a tap are two float4 loads.
#include <type_traits>

#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

// Register-tiled variant: a thread owns 8 data channels (and the matching 8
// gate channels) of one row segment of XS output tokens.  Its 9 taps x 16
// channels of weights and its biases are loaded once; a 3 x 3 window of input
// vectors slides along the row, so each new output token loads one new input
// column (3 rows) instead of all 9 taps.  Taps are summed in (ky, kx) order
// with zero padding, then the bias, as the reference accumulates.
template <int XS>
__global__ __launch_bounds__(64) void dwglu_row_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                       const float * __restrict__ wt, const float * __restrict__ bias,
                                                       f16 * __restrict__ out, int64_t ldo, int Hh, int Ww, int F) {
    const int G = F / 8;
    const int g = blockIdx.x * 64 + threadIdx.x;
    const int nseg = (Ww + XS - 1) / XS;
    const int y = blockIdx.y / nseg, seg = blockIdx.y - (blockIdx.y / nseg) * nseg;
    const int b = blockIdx.z;
    if (g >= G) return;
    const int c0 = g * 8, E = 2 * F;
    float wd[9][8], wg[9][8];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const float4 * wp = reinterpret_cast<const float4 *>(wt + (int64_t)k * E + c0);
        const float4 * wq = reinterpret_cast<const float4 *>(wt + (int64_t)k * E + F + c0);
        const float4 a0 = wp[0], a1 = wp[1], b0 = wq[0], b1 = wq[1];
        wd[k][0] = a0.x; wd[k][1] = a0.y; wd[k][2] = a0.z; wd[k][3] = a0.w;
        wd[k][4] = a1.x; wd[k][5] = a1.y; wd[k][6] = a1.z; wd[k][7] = a1.w;
        wg[k][0] = b0.x; wg[k][1] = b0.y; wg[k][2] = b0.z; wg[k][3] = b0.w;
        wg[k][4] = b1.x; wg[k][5] = b1.y; wg[k][6] = b1.z; wg[k][7] = b1.w;
    }
    float bd[8], bg[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        bd[e] = bias[c0 + e];
        bg[e] = bias[F + c0 + e];
    }
    const f16 * xb = x + (int64_t)b * Hh * Ww * ldx + c0;
    f16 * ob = out + (int64_t)b * Hh * Ww * ldo + c0;
    const int x0 = seg * XS;
    f16x8 vd[3][3], vg[3][3];  // [row ky][column slot]
    auto load = [&](int ky, int xx, int slot) {
        const int yy = y + ky - 1;
        if (yy >= 0 && yy < Hh && xx >= 0 && xx < Ww) {
            const f16 * p = xb + ((int64_t)yy * Ww + xx) * ldx;
            vd[ky][slot] = *reinterpret_cast<const f16x8 *>(p);
            vg[ky][slot] = *reinterpret_cast<const f16x8 *>(p + F);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) vd[ky][slot][e] = vg[ky][slot][e] = (f16)0.0f;
        }
    };
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
        load(ky, x0 - 1, 0);
        load(ky, x0, 1);
    }
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int xx = x0 + i;
        if (xx < Ww) {
#pragma unroll
            for (int ky = 0; ky < 3; ++ky) load(ky, xx + 1, (i + 2) % 3);
            float ad[8], ag[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) ad[e] = ag[e] = 0.0f;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const int slot = (i + kx) % 3;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        ad[e] += (float)vd[ky][slot][e] * wd[ky * 3 + kx][e];
                        ag[e] += (float)vg[ky][slot][e] * wg[ky * 3 + kx][e];
                    }
                }
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = ad[e] + bd[e];
                const float gt = ag[e] + bg[e];
                o[e] = (f16)(d * silu_fast(gt));
            }
            *reinterpret_cast<f16x8 *>(ob + ((int64_t)y * Ww + xx) * ldo) = o;
        }
    }
}

// Pipelined variant: a thread owns 4 data channels (and the matching 4 gate
// channels) of a row segment of XS output tokens, so its weights (9 taps x 8
// channels, fp32) and input window fit in ~150 VGPRs (three waves per SIMD
// instead of two).  The window is a ring of 3 + PD input columns: the column
// token i + PD needs is requested before token i's arithmetic, so each load
// has PD tokens' worth of math to land behind.  Taps are summed in (ky, kx)
// order with zero padding, then the bias, as in dwglu_row_kernel (same
// per-channel arithmetic, same results).
template <int XS, int PD = 1>
__global__ __launch_bounds__(64) void dwglu_pipe_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                        const float * __restrict__ wt,
                                                        const float * __restrict__ bias, f16 * __restrict__ out,
                                                        int64_t ldo, int Hh, int Ww, int F) {
    const int G = F / 4;
    const int g = blockIdx.x * 64 + threadIdx.x;
    const int nseg = (Ww + XS - 1) / XS;
    const int y = blockIdx.y / nseg, seg = blockIdx.y - (blockIdx.y / nseg) * nseg;
    const int b = blockIdx.z;
    if (g >= G) return;
    const int c0 = g * 4, E = 2 * F;
    float wd[9][4], wg[9][4];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const float4 a = *reinterpret_cast<const float4 *>(wt + (int64_t)k * E + c0);
        const float4 q = *reinterpret_cast<const float4 *>(wt + (int64_t)k * E + F + c0);
        wd[k][0] = a.x; wd[k][1] = a.y; wd[k][2] = a.z; wd[k][3] = a.w;
        wg[k][0] = q.x; wg[k][1] = q.y; wg[k][2] = q.z; wg[k][3] = q.w;
    }
    const float4 bdv = *reinterpret_cast<const float4 *>(bias + c0);
    const float4 bgv = *reinterpret_cast<const float4 *>(bias + F + c0);
    const float bd[4] = {bdv.x, bdv.y, bdv.z, bdv.w}, bg[4] = {bgv.x, bgv.y, bgv.z, bgv.w};
    const f16 * xb = x + (int64_t)b * Hh * Ww * ldx + c0;
    f16 * ob = out + (int64_t)b * Hh * Ww * ldo + c0;
    const int x0 = seg * XS;
    constexpr int NS = 3 + PD;  // ring of input columns: column x0 - 1 + j lives in slot j % NS
    f16x4 vd[3][NS], vg[3][NS];
    auto load = [&](int ky, int xx, int slot) {
        const int yy = y + ky - 1;
        if (yy >= 0 && yy < Hh && xx >= 0 && xx < Ww) {
            const f16 * p = xb + ((int64_t)yy * Ww + xx) * ldx;
            vd[ky][slot] = *reinterpret_cast<const f16x4 *>(p);
            vg[ky][slot] = *reinterpret_cast<const f16x4 *>(p + F);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) vd[ky][slot][e] = vg[ky][slot][e] = (f16)0.0f;
        }
    };
    // columns x0 - 1 .. x0 + PD before the first token
#pragma unroll
    for (int j = 0; j < 2 + PD; ++j)
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) load(ky, x0 - 1 + j, j);
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int xx = x0 + i;
        if (xx < Ww) {
            // the column token i + PD needs (x0 + i + PD + 1), PD tokens ahead
            if (i + PD < XS) {
#pragma unroll
                for (int ky = 0; ky < 3; ++ky) load(ky, xx + PD + 1, (i + PD + 2) % NS);
            }
            float ad[4], ag[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) ad[e] = ag[e] = 0.0f;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const int slot = (i + kx) % NS;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ad[e] += (float)vd[ky][slot][e] * wd[ky * 3 + kx][e];
                        ag[e] += (float)vg[ky][slot][e] * wg[ky * 3 + kx][e];
                    }
                }
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = ad[e] + bd[e];
                const float gt = ag[e] + bg[e];
                o[e] = (f16)(d * silu_fast(gt));
            }
            *reinterpret_cast<f16x4 *>(ob + ((int64_t)y * Ww + xx) * ldo) = o;
        }
    }
}

#define SANA_LDS(p) ((__attribute__((address_space(3))) void *)(p))
constexpr int kDwStripW = 32;                // output tokens per strip row
constexpr int kDwStripC = 32;                // data channels per workgroup
constexpr int64_t kDwStripMinTokens = 1024;  // tokens per launch from which the strip kernel is used

// LDS-tiled variant for grids too small for tall strips (below): a workgroup
// of 256 threads takes a TH x 32 tile of output tokens and 32 data channels
// (with the matching 32 gate channels).  The (TH + 2) x 34 input tokens of the
// tile and its one-token halo are copied into LDS with global_load_lds_dwordx4
// (two planes, data and gate, of 64-byte token rows, in chunk order so each
// wave instruction fills one contiguous KiB) in one go, 26 KB at TH = 4, and
// one barrier later the tile is computed.  Thread (column x, channel
// quad q) then slides a 3 x 3 window down its column of TH outputs, reading
// one new input row (3 columns x 8 bytes of data and of gate) from LDS per
// output; lanes 8 apart read consecutive tokens, so a wave's 8-byte reads
// cover 256 contiguous bytes (no bank conflicts).  Halo positions outside the
// grid are loaded from clamped addresses and zeroed in registers.  Taps are
// summed in (ky, kx) order with zero padding, then the bias, as in
// dwglu_row_kernel (same per-channel arithmetic, same results).
template <int TH>
struct DwTile {
    static constexpr int ROWS = TH + 2, COLS = kDwStripW + 2, TOK = ROWS * COLS;
    static constexpr int CHUNKS = 2 * TOK * (kDwStripC * 2 / 16);  // 16-byte chunks, both planes
    static constexpr int INSTR = (CHUNKS + 63) / 64;              // wave DMA instructions
    static constexpr int PLANE = TOK * kDwStripC * 2;              // bytes per plane
    static constexpr int LDS = INSTR * 1024;                      // the last instruction's tail lanes land past the planes
};

template <int TH>
__global__ __launch_bounds__(256) void dwglu_tile_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                         const float * __restrict__ wt,
                                                         const float * __restrict__ bias, f16 * __restrict__ out,
                                                         int64_t ldo, int Hh, int Ww, int F) {
    using T = DwTile<TH>;
    __shared__ __attribute__((aligned(16))) unsigned char lds[T::LDS];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    // Workgroups are dealt round-robin to the 8 XCDs (each with its own L2).
    // Tiles vary fastest, so with a multiple of 8 tiles the channel groups that
    // share the 128-byte lines of a token (c0 and c0 + 32) run on one XCD; and
    // XCD x takes a contiguous range of tiles in column-band-major order, so
    // the tiles above and below one another, which share two halo rows, mostly
    // run on the same XCD too.
    const int c0 = blockIdx.y * kDwStripC;
    const int nty = (Hh + TH - 1) / TH;
    const int nt = (int)gridDim.x, per = nt / 8, id = (int)blockIdx.x;
    const int o = id < per * 8 ? (id % 8) * per + id / 8 : id;
    const int ty0 = (o % nty) * TH, tx0 = (o / nty) * kDwStripW;
    const int b = blockIdx.z;
    const f16 * xb = x + (int64_t)b * Hh * Ww * ldx + c0;
    // 1. staging: chunk g = plane * (TOK * 4) + token * 4 + part -> LDS byte 16 g
    for (int i = wid; i < T::INSTR; i += 4) {
        const int g = min(i * 64 + lane, T::CHUNKS - 1);
        const int plane = g / (T::TOK * 4), within = g - plane * (T::TOK * 4);
        const int tok = within >> 2, part = within & 3;
        const int r = tok / T::COLS, cc = tok - r * T::COLS;
        const int yy = min(max(ty0 + r - 1, 0), Hh - 1), xx = min(max(tx0 + cc - 1, 0), Ww - 1);
        const f16 * src = xb + ((int64_t)yy * Ww + xx) * ldx + plane * F + part * 8;
        __builtin_amdgcn_global_load_lds(static_cast<const void *>(src), SANA_LDS(lds + i * 1024), 16, 0, 0);
    }
    // weights and bias of this thread's 4 channels (in flight with the staging)
    const int q = tid & 7, xo = tid >> 3;  // channel quad, output column in the tile
    const int c = c0 + 4 * q, E = 2 * F;
    float wd[9][4], wg[9][4];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const float4 a = *reinterpret_cast<const float4 *>(wt + (int64_t)k * E + c);
        const float4 g4 = *reinterpret_cast<const float4 *>(wt + (int64_t)k * E + F + c);
        wd[k][0] = a.x; wd[k][1] = a.y; wd[k][2] = a.z; wd[k][3] = a.w;
        wg[k][0] = g4.x; wg[k][1] = g4.y; wg[k][2] = g4.z; wg[k][3] = g4.w;
    }
    const float4 bdv = *reinterpret_cast<const float4 *>(bias + c);
    const float4 bgv = *reinterpret_cast<const float4 *>(bias + F + c);
    const float bd[4] = {bdv.x, bdv.y, bdv.z, bdv.w}, bg[4] = {bgv.x, bgv.y, bgv.z, bgv.w};
    __builtin_amdgcn_s_waitcnt((0 & 15) | (7 << 4) | (15 << 8) | (0 << 14));  // vmcnt(0): this wave's DMA landed
    __syncthreads();

    // 2. the column's outputs; input column j of the window is tile column xo + j
    const int ox = tx0 + xo;
    bool colok[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int ix = ox + j - 1;
        colok[j] = ix >= 0 && ix < Ww;
    }
    const f16 * dp = reinterpret_cast<const f16 *>(lds);
    const f16 * gp = reinterpret_cast<const f16 *>(lds + T::PLANE);
    f16x4 vd[3][3], vg[3][3];  // [window row][column]
    auto load_row = [&](int slot, int r) {  // tile-local input row r (0 .. TH + 1)
        const int iy = ty0 + r - 1;
        const bool rok = iy >= 0 && iy < Hh;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int off = ((r * T::COLS + xo + j) * kDwStripC + 4 * q);
            f16x4 d4 = *reinterpret_cast<const f16x4 *>(dp + off);
            f16x4 g4 = *reinterpret_cast<const f16x4 *>(gp + off);
            if (!(rok && colok[j])) {
#pragma unroll
                for (int e = 0; e < 4; ++e) d4[e] = g4[e] = (f16)0.0f;
            }
            vd[slot][j] = d4;
            vg[slot][j] = g4;
        }
    };
    load_row(0, 0);
    load_row(1, 1);
#pragma unroll
    for (int r = 0; r < TH; ++r) {
        load_row((r + 2) % 3, r + 2);
        const int oy = ty0 + r;
        if (oy >= Hh || ox >= Ww) continue;
        float ad[4], ag[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ad[e] = ag[e] = 0.0f;
#pragma unroll
        for (int ky = 0; ky < 3; ++ky)
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int slot = (r + ky) % 3;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ad[e] += (float)vd[slot][kx][e] * wd[ky * 3 + kx][e];
                    ag[e] += (float)vg[slot][kx][e] * wg[ky * 3 + kx][e];
                }
            }
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = ad[e] + bd[e];
            const float gt = ag[e] + bg[e];
            o[e] = (f16)(d * silu_fast(gt));
        }
        *reinterpret_cast<f16x4 *>(out + ((int64_t)(b * Hh + oy) * Ww + ox) * ldo + c) = o;
    }
}

// LDS strip variant for long sequences: a workgroup of 256 threads walks a
// strip of SH x 32 output tokens and 32 data (+ 32 gate) channels down the
// grid, one output row per step.  Input rows (34 tokens with the halo
// columns; data and gate planes of 64-byte token rows: 4352 bytes) stream
// into a ring of kDwStripRing LDS slots by global_load_lds_dwordx4, P rows
// ahead of the first row a step consumes, so the DMA of later rows is in
// flight while a row's arithmetic runs and each input row is fetched once per
// strip (tiles of TH rows fetch their two halo rows again: 10 rows for 8 at
// TH = 8).  Each wave moves 68 of a row's 272 16-byte chunks (two
// instructions, the second on 4 lanes), so every wave issues the same two DMA
// instructions per row and its own vmcnt tracks a row's arrival.  Thread
// (column x, channel quad q) keeps a 3 x 3 window of 4-channel vectors in
// registers and reads one new input row (3 columns x 8 bytes of data and of
// gate) from LDS per step; lanes 8 apart read consecutive tokens, so a wave's
// 8-byte reads cover 256 contiguous bytes (no bank conflicts).  Halo
// positions outside the grid are loaded from clamped addresses and zeroed in
// registers.  Taps are summed in (ky, kx) order with zero padding, then the
// bias, as in dwglu_row_kernel (same per-channel arithmetic, same results).
constexpr int kDwStripRow = 2 * (kDwStripW + 2) * kDwStripC * 2;  // bytes per staged input row (both planes)
constexpr int kDwStripChunks = kDwStripRow / 16;                // 272 chunks: 68 per wave
constexpr int kDwStripRing = 8;                                 // LDS row slots

// s_waitcnt vmcnt(2 k), k = input rows whose DMA may stay in flight (gfx9
// encoding, the other counters unconstrained)
template <int K>
SANA_DEV void dw_wait_rows() {
    static_assert(2 * K < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(((2 * K) & 15) | (7 << 4) | (15 << 8) | (((2 * K) >> 4) << 14));
}
template <int KMAX>
SANA_DEV void dw_wait_rows_upto(int k) {
    if constexpr (KMAX > 0) {
        if (k >= KMAX) {
            dw_wait_rows<KMAX>();
            return;
        }
        dw_wait_rows_upto<KMAX - 1>(k);
    } else {
        dw_wait_rows<0>();
    }
}

template <int SH, int P>
__global__ __launch_bounds__(256) void dwglu_strip_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                          const float * __restrict__ wt,
                                                          const float * __restrict__ bias, f16 * __restrict__ out,
                                                          int64_t ldo, int Hh, int Ww, int F) {
    // the prologue's rows 0 .. P - 1 take distinct slots; later, rows j + 2 ..
    // j + P - 1 are resident or in flight when row j + P is requested into the
    // slot of row j + P - kDwStripRing, which step j - 1 finished reading
    static_assert(P >= 3 && P <= kDwStripRing, "prefetch distance against the ring");
    __shared__ __attribute__((aligned(16))) unsigned char lds[kDwStripRing * kDwStripRow + 3 * 1024];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    // Workgroups are dealt round-robin to the 8 XCDs (each with its own L2).
    // Strips vary fastest, so with a multiple of 8 strips the channel groups
    // that share the 128-byte lines of a token (c0 and c0 + 32) run on one XCD;
    // and XCD x takes a contiguous range of strips in column-band-major order,
    // so strips above and below one another, which share a halo row, mostly
    // run on the same XCD too.
    const int c0 = blockIdx.y * kDwStripC;
    const int nsy = (Hh + SH - 1) / SH;
    const int nt = (int)gridDim.x, per = nt / 8, id = (int)blockIdx.x;
    const int o = id < per * 8 ? (id % 8) * per + id / 8 : id;
    const int sy0 = (o % nsy) * SH, tx0 = (o / nsy) * kDwStripW;
    const int b = blockIdx.z;
    const int nout = min(SH, Hh - sy0), rows = nout + 2;  // output rows; input rows sy0 - 1 .. sy0 + nout
    const f16 * xb = x + (int64_t)b * Hh * Ww * ldx + c0;
    // this lane's chunks of an input row: g0 = 68 wid + lane, g1 = g0 + 64 (lanes < 4)
    auto chunk_off = [&](int g) -> int64_t {
        const int plane = g / (kDwStripChunks / 2), within = g - plane * (kDwStripChunks / 2);
        const int tok = within >> 2, part = within & 3;
        const int xx = min(max(tx0 + tok - 1, 0), Ww - 1);
        return (int64_t)xx * ldx + plane * F + part * 8;
    };
    const int gw = (kDwStripChunks / 4) * wid;
    const int64_t off0 = chunk_off(gw + lane), off1 = chunk_off(gw + 64 + (lane & 3));
    auto issue_row = [&](int r) {  // strip-local input row r -> ring slot r % kDwStripRing
        const int yy = min(max(sy0 + r - 1, 0), Hh - 1);
        const f16 * rp = xb + (int64_t)yy * Ww * ldx;
        unsigned char * slot = lds + (r % kDwStripRing) * kDwStripRow + gw * 16;
        __builtin_amdgcn_global_load_lds(static_cast<const void *>(rp + off0), SANA_LDS(slot), 16, 0, 0);
        if (lane < 4)
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(rp + off1), SANA_LDS(slot + 1024), 16, 0, 0);
    };
    // The workgroup's weights and biases (9 taps x 32 data + 32 gate channels,
    // then the two bias rows: 160 16-byte chunks) go to LDS by the same DMA,
    // ahead of the rows: every global access of the kernel is then a DMA or a
    // store, so the only vmcnt waits are the row waits below (a weight kept in
    // a VGPR from a global load would make the compiler wait for every
    // outstanding DMA before its first use in each step).
    float * wl = reinterpret_cast<float *>(lds + kDwStripRing * kDwStripRow);  // [10][2][32]: taps 0..8, bias
    if (wid < 3) {
        const int i = min(wid * 64 + lane, 159);
        const int k = i >> 4, plane = (i >> 3) & 1, grp = i & 7;
        const float * src = (k < 9 ? wt + (int64_t)k * (2 * F) : bias) + plane * F + c0 + 4 * grp;
        __builtin_amdgcn_global_load_lds(static_cast<const void *>(src), SANA_LDS(lds + kDwStripRing * kDwStripRow + wid * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < P; ++r)
        if (r < rows) issue_row(r);
    const int q = tid & 7, xo = tid >> 3;  // channel quad, output column in the strip
    const int c = c0 + 4 * q;
    const int ox = tx0 + xo;
    bool colok[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int ix = ox + j - 1;
        colok[j] = ix >= 0 && ix < Ww;
    }
    f16x4 vd[3][3], vg[3][3];  // [window row][column]
    auto load_row = [&](int wslot, int r) {  // strip-local input row r from its ring slot
        const int iy = sy0 + r - 1;
        const bool rok = iy >= 0 && iy < Hh;
        const f16 * dp = reinterpret_cast<const f16 *>(lds + (r % kDwStripRing) * kDwStripRow);
        const f16 * gp = dp + kDwStripRow / 4;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int off = (xo + j) * kDwStripC + 4 * q;
            f16x4 d4 = *reinterpret_cast<const f16x4 *>(dp + off);
            f16x4 g4 = *reinterpret_cast<const f16x4 *>(gp + off);
            if (!(rok && colok[j])) {
#pragma unroll
                for (int e = 0; e < 4; ++e) d4[e] = g4[e] = (f16)0.0f;
            }
            vd[wslot][j] = d4;
            vg[wslot][j] = g4;
        }
    };
    // rows 0 and 1 have landed (every row requested after them may stay in flight)
    __builtin_amdgcn_sched_barrier(0);
    dw_wait_rows_upto<P - 2>(min(P, rows) - 2);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // (read as 16-byte f16x8 words, the type of the row reads: the row waits
    // above already cover these DMAs, and with that type the compiler adds no
    // wait of its own for every DMA in flight)
    float wd[9][4], wg[9][4], bd[4], bg[4];
    auto wload = [&](int row, float (&dst)[4]) {
        const f16x8 v = *reinterpret_cast<const f16x8 *>(wl + row * 32 + 4 * q);
        __builtin_memcpy(dst, &v, 16);
    };
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        wload(k * 2 + 0, wd[k]);
        wload(k * 2 + 1, wg[k]);
    }
    wload(18, bd);
    wload(19, bg);
    load_row(0, 0);
    load_row(1, 1);
#pragma unroll
    for (int j = 0; j < SH; ++j) {
        if (j >= nout) continue;  // uniform: the last strip of a grid whose height is not a multiple of SH
        // row j + 2 has landed in every wave, and every LDS read issued before
        // (the slot the next DMA takes included) has returned
        __builtin_amdgcn_sched_barrier(0);
        dw_wait_rows_upto<P - 3>(min(j + P - 1, rows - 1) - (j + 2));
        __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (j + P < rows) issue_row(j + P);
        load_row((j + 2) % 3, j + 2);
        const int oy = sy0 + j;
        if (ox < Ww) {
            float ad[4], ag[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) ad[e] = ag[e] = 0.0f;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const int slot = (j + ky) % 3;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ad[e] += (float)vd[slot][kx][e] * wd[ky * 3 + kx][e];
                        ag[e] += (float)vg[slot][kx][e] * wg[ky * 3 + kx][e];
                    }
                }
            f16x4 ov;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = ad[e] + bd[e];
                const float gt = ag[e] + bg[e];
                ov[e] = (f16)(d * silu_fast(gt));
            }
            *reinterpret_cast<f16x4 *>(out + ((int64_t)(b * Hh + oy) * Ww + ox) * ldo + c) = ov;
        }
    }
}

// Scalar variant for channel counts that are not a multiple of 8.
__global__ __launch_bounds__(256) void dwglu_scalar_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                           const float * __restrict__ wt,
                                                           const float * __restrict__ bias, f16 * __restrict__ out,
                                                           int64_t ldo, int B, int Hh, int Ww, int F) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)B * Hh * Ww * F;
    if (gid >= total) return;
    const int c = (int)(gid % F);
    const int64_t m = gid / F;
    const int xx = (int)(m % Ww);
    const int64_t r = m / Ww;
    const int y = (int)(r % Hh);
    const int b = (int)(r / Hh);
    const int E = 2 * F;
    float ad = 0.0f, ag = 0.0f;
    for (int ky = 0; ky < 3; ++ky) {
        const int iy = y + ky - 1;
        if (iy < 0 || iy >= Hh) continue;
        for (int kx = 0; kx < 3; ++kx) {
            const int ix = xx + kx - 1;
            if (ix < 0 || ix >= Ww) continue;
            const f16 * px = x + (((int64_t)b * Hh + iy) * Ww + ix) * ldx;
            ad += (float)px[c] * wt[(ky * 3 + kx) * E + c];
            ag += (float)px[F + c] * wt[(ky * 3 + kx) * E + F + c];
        }
    }
    const float d = ad + bias[c], g = ag + bias[F + c];
    out[m * ldo + c] = (f16)(d * silu_f(g));
}

}  // namespace

hipError_t dwconv_glu(const half_t * x, int64_t ldx, const float * wt, const float * bias, half_t * out, int64_t ldo,
                      int B, int Hh, int Ww, int F, hipStream_t s) {
    if (B <= 0 || Hh <= 0 || Ww <= 0 || F <= 0 || ldx < 2 * (int64_t)F || ldo < F || !bias || !wt)
        return hipErrorInvalidValue;
    const bool vec = F % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       reinterpret_cast<uintptr_t>(wt)) & 15) == 0;
    const f16 * xx = reinterpret_cast<const f16 *>(x);
    f16 * oo = reinterpret_cast<f16 *>(out);
    if (vec) {
        const int64_t tokens = (int64_t)B * Hh * Ww;
        if (B > 65535) return hipErrorInvalidValue;
        auto launch = [&](auto xs_tag, const char * name, auto pipe_tag) {
            constexpr int XS = decltype(xs_tag)::value;
            constexpr bool PIPE = decltype(pipe_tag)::value;
            const int64_t nseg = (Ww + XS - 1) / XS;
            if ((int64_t)Hh * nseg > 2147483647) return hipErrorInvalidValue;
            note_kernel(name);
            if constexpr (PIPE)
                hipLaunchKernelGGL((dwglu_pipe_kernel<XS>), dim3((F / 4 + 63) / 64, (unsigned)(Hh * nseg), B),
                                   dim3(64), 0, s, xx, ldx, wt, bias, oo, ldo, Hh, Ww, F);
            else
                hipLaunchKernelGGL((dwglu_row_kernel<XS>), dim3((F / 8 + 63) / 64, (unsigned)(Hh * nseg), B),
                                   dim3(64), 0, s, xx, ldx, wt, bias, oo, ldo, Hh, Ww, F);
            return hipSuccess;
        };
        using P = std::true_type;
        hipError_t e;
        if (F % 4 == 0 && ((reinterpret_cast<uintptr_t>(bias) & 15) == 0)) {
            // Pipelined 4-channel kernel (bit-identical to the 8-channel row
            // kernel), row segment by token count; alone on the GPU, 2880
            // channels, inputs cycled through buffers past the last-level
            // cache, us (8-channel row kernel at its best XS in brackets):
            //   tokens           XS = 4    8      16     32
            //   1024 (32x32)     9.55     9.86   11.23  18.09   (10.28)
            //   4096 (64x64)     28.50    24.17  22.08  27.42   (24.34)
            //   9216 (96x96)     77.06    63.19  59.30  66.31   (61.53)
            //   16384 (128x128)  139.89   112.18 99.65  92.83   (97.83)
            // The VAE's power-of-two channel counts put the rows of the token
            // grid a power of two of bytes apart (2F halves per token), and
            // there the row kernel with 16-token segments wins from 16M
            // outputs on: F = 2048 at 16384 tokens 62.6 us against 65.2 /
            // 71.8 (pipe16 / pipe32), F = 4096 at 4096 tokens 27.2 against
            // 30.1 / 29.7; F = 4096 at 1024 tokens pipe8 10.5 against pipe4
            // 11.7.  F = 2048 at 4096 tokens keeps pipe16 (17.0 against 19.6).
            const bool pow2 = (F & (F - 1)) == 0;
            if (tokens >= kDwStripMinTokens && F % kDwStripC == 0 && !pow2 && F / kDwStripC <= 65535) {
                // LDS strip kernel: the tallest strip (32, 16 or 8 rows) that
                // still makes >= 720 workgroups, else 4 x 32 tiles staged whole
                // (alone on the GPU, 2880 channels, inputs cycled past the
                // last-level cache, us):
                //   grid      SH,P = 32,5   32,4   16,4   16,5   8,4    4,4     tiles TH = 4 / 8
                //   32x32            -      -      12.68  -      10.07  8.25    8.92 / 11.77
                //   64x64            26.93  29.54  21.29  21.57  23.52  26.16   26.30 / 25.69
                //   128x128          71.26  71.88  75.18  72.57  78.67  86.13   86.96 / 80.15
                // (64-row strips spill the window registers; a prefetch of 3 rows
                // is 5-7 % slower than 4-5.)  At 32 x 32, though, the 1024 px
                // forward with the two CFG branches' launches side by side ran
                // 4.935 ms with 4-row strips against 4.902 with 4-row tiles in one
                // process (bit-identical), so grids that small keep the tiles.
                auto strip = [&](auto sh_tag, auto p_tag, const char * name) {
                    constexpr int SH = decltype(sh_tag)::value, PF = decltype(p_tag)::value;
                    const int64_t strips = (int64_t)((Hh + SH - 1) / SH) * ((Ww + kDwStripW - 1) / kDwStripW);
                    if (strips > 2147483647) return hipErrorInvalidValue;
                    note_kernel(name);
                    hipLaunchKernelGGL((dwglu_strip_kernel<SH, PF>), dim3((unsigned)strips, F / kDwStripC, B), dim3(256),
                                       0, s, xx, ldx, wt, bias, oo, ldo, Hh, Ww, F);
                    return hipSuccess;
                };
                auto wgs = [&](int sh) {
                    return (int64_t)((Hh + sh - 1) / sh) * ((Ww + kDwStripW - 1) / kDwStripW) * (F / kDwStripC) * B;
                };
                using I4 = std::integral_constant<int, 4>;
                if (wgs(32) >= 720)
                    e = strip(std::integral_constant<int, 32>{}, std::integral_constant<int, 5>{},
                              "dwglu_strip_kernel<32, 5>");
                else if (wgs(16) >= 720)
                    e = strip(std::integral_constant<int, 16>{}, I4{}, "dwglu_strip_kernel<16, 4>");
                else if (wgs(8) >= 720)
                    e = strip(std::integral_constant<int, 8>{}, I4{}, "dwglu_strip_kernel<8, 4>");
                else {
                    const int64_t tiles = (int64_t)((Hh + 3) / 4) * ((Ww + kDwStripW - 1) / kDwStripW);
                    if (tiles > 2147483647) return hipErrorInvalidValue;
                    note_kernel("dwglu_tile_kernel<4>");
                    hipLaunchKernelGGL((dwglu_tile_kernel<4>), dim3((unsigned)tiles, F / kDwStripC, B), dim3(256), 0, s,
                                       xx, ldx, wt, bias, oo, ldo, Hh, Ww, F);
                    e = hipSuccess;
                }
            } else if (pow2 && tokens * F >= (int64_t)1 << 24)
                e = launch(std::integral_constant<int, 16>{}, "dwglu_row_kernel<16>", std::false_type{});
            else if (tokens <= 1024 && F >= 4096)
                e = launch(std::integral_constant<int, 8>{}, "dwglu_pipe_kernel<8>", P{});
            else if (tokens <= 1024) e = launch(std::integral_constant<int, 4>{}, "dwglu_pipe_kernel<4>", P{});
            else if (tokens <= 2048) e = launch(std::integral_constant<int, 8>{}, "dwglu_pipe_kernel<8>", P{});
            else if (tokens < 12288) e = launch(std::integral_constant<int, 16>{}, "dwglu_pipe_kernel<16>", P{});
            else e = launch(std::integral_constant<int, 32>{}, "dwglu_pipe_kernel<32>", P{});
        } else {
            // 8-channel row kernel: row segment by token count (inputs cycled)
            //   tokens           XS = 4     8        16
            //   1024 (32x32)     11.2 us    12.1     19.0
            //   2048 (2x32x32)   18.8       18.4     23.0
            //   4096 (64x64)     35.9       32.3     32.6
            //   16384 (128x128)  127.4      112.6    102.0
            using R = std::false_type;
            if (tokens <= 1024) e = launch(std::integral_constant<int, 4>{}, "dwglu_row_kernel<4>", R{});
            else if (tokens < 12288) e = launch(std::integral_constant<int, 8>{}, "dwglu_row_kernel<8>", R{});
            else e = launch(std::integral_constant<int, 16>{}, "dwglu_row_kernel<16>", R{});
        }
        if (e != hipSuccess) return e;
    } else {
        const int64_t total = (int64_t)B * Hh * Ww * F;
        note_kernel("dwglu_scalar_kernel");
        hipLaunchKernelGGL(dwglu_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, xx, ldx, wt,
                           bias, oo, ldo, B, Hh, Ww, F);
    }
    return hipGetLastError();
}

}  // namespace sana
