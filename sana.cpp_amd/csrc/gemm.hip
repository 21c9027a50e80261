// K1: MFMA GEMM for every dense projection of the DiT (QKV, attention output,
// cross-attention q/k/v/out, Mix-FFN inverted/point 1x1 convs, caption MLP).
//
// C[m, n] = sum_k A[m, k] * W[n, k], fp16 operands, fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  A (activations, token-major) and W (weights,
// PyTorch [out, in] order) are both K-contiguous, so each MFMA lane's operand
// (8 consecutive k of one row) is a single 16-byte LDS read.
//
// Data movement (gfx950):
//   * HBM/L2 -> LDS with global_load_lds_dwordx4: each wave instruction moves
//     8 rows x 64 k (1 KB) straight into LDS without passing through VGPRs.
//   * A STAGES-deep ring of LDS k-tiles (BK = 64): when tile kt is done its
//     stage is refilled with tile kt+STAGES, so each load has STAGES-1 tiles
//     of MFMA work to land.  Completion is tracked with an explicit vmcnt
//     wait (the loads of later tiles stay outstanding) and one s_barrier per
//     k-tile, placed after the tile's last MFMAs are issued.
//   * LDS rows are 128 bytes; 16-byte chunk c of row r is stored in slot
//     c ^ ((r >> 1) & 7).  The DMA writes lane l to slot l & 7 of row l >> 3 of
//     its 8-row block, so lane l fetches the chunk that maps there.  gfx950's
//     LDS serves a 16-byte read 16 lanes (256 bytes, all 64 banks) per cycle;
//     an MFMA operand read of 16 consecutive rows at one chunk then hits 16
//     distinct 16-byte bank groups (row parity picks the half of the 256-byte
//     window, (r >> 1) & 7 the group within it): no bank conflicts.  The
//     slot c ^ (r & 7) conflicts two ways (rows r and r + 8 share a group).
//   * Epilogue staged through LDS: the MFMA computes the transposed tile, so
//     each lane holds runs of 4 consecutive columns of one row and writes
//     them to LDS as one 16-byte (fp32) or 8-byte (fp16) store; then every
//     thread moves 8 consecutive columns with 16-byte global accesses.
//     Outputs that are fp16 only are rounded in registers and staged as fp16
//     (one pass for every tile shape).
//
// The workgroup -> tile map is XCD-aware: gfx950 deals workgroups round-robin
// to 8 XCDs (each with its own L2), so workgroup id i goes to position
// (i % 8) * (T / 8) + i / 8 of a grouped tile order (8 row panels at a time,
// column by column): the tiles one XCD runs concurrently form a compact 2-D
// block whose A and W panels are shared through its L2.
//
// Fused epilogues (reference ops they replace):
//   store   : bias (+SiLU | +GELU-tanh), fp16 and/or fp32 out
//             (linear_3d_lastdim src/common_ops.cpp:177-209, silu src/tensor.cpp:551-555,
//              gelu_tanh src/transformer_ops.cpp:15-18)
//   residual: x += gate * (acc + bias), optional fp16 copy of the new x
//             (mul_inplace_broadcast_lastdim + add_inplace, src/tensor.cpp:101-160)
//   V^T     : transposed per-batch store of the cross-attention values.
#include <string>

#include "hip_common.h"
#include "kernels.h"

#define SANA_LDS(p) ((__attribute__((address_space(3))) void *)(p))

namespace sana {
namespace gemm_detail {

constexpr int kBK = 64;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
SANA_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0): every LDS read of this wave has returned.
SANA_DEV void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

template <int BM, int BN, int WM, int WN, int STAGES>
struct Cfg {
    static constexpr int NW = WM * WN;
    static constexpr int NT = 64 * NW;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int TM = WTM / 32, TN = WTN / 32;
    static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int A_LOADS = BM / 8 / NW, B_LOADS = BN / 8 / NW;  // wave instructions per stage
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr int CPAD = 4;                                      // fp32 epilogue row padding
    // The fp32 epilogue tile is staged in LDS: whole when it fits in the operand
    // ring or in 80 KB (two workgroups per CU), else one wave row (WTM rows) per pass.
    static constexpr int RING_BYTES = STAGES * STAGE_BYTES;
    static constexpr int EPI_ROWS =
        (BM * (BN + CPAD) * 4 <= (RING_BYTES > 80 * 1024 ? RING_BYTES : 80 * 1024)) ? BM : WTM;
    static constexpr int EPI_BYTES = EPI_ROWS * (BN + CPAD) * 4;
    static constexpr int LDS_BYTES = (RING_BYTES > EPI_BYTES) ? RING_BYTES : EPI_BYTES;
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "tile rows must split into 8-row wave loads");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
    static_assert(LOADS * STAGES < 64, "vmcnt range");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// Wait until at most `keep` stages (0 <= keep < STAGES) of this wave's loads are outstanding.
template <int LOADS, int STAGES>
SANA_DEV void wait_stages(int keep) {
    if constexpr (STAGES >= 4) {
        if (keep >= 3) { wait_vmcnt<3 * LOADS>(); return; }
    }
    if constexpr (STAGES >= 3) {
        if (keep >= 2) { wait_vmcnt<2 * LOADS>(); return; }
    }
    if (keep >= 1) { wait_vmcnt<LOADS>(); return; }
    wait_vmcnt<0>();
}

// CONV: 0 plain A rows; 1 implicit 3x3 conv over a zero-bordered NHWC input;
// 2 the same over the nearest-2x upsample of the input (GemmParams::conv).
template <int BM, int BN, int WM, int WN, int STAGES, int MODE, int SCHED, int ACT, int CONV = 0>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmParams p_in) {
    using G = Cfg<BM, BN, WM, WN, STAGES>;
    // product blockIdx.y of a batched launch (plain stores only)
    GemmParams p = p_in;
    if constexpr (MODE == kGemmStore && CONV == 0) {
        const int z = blockIdx.y;
        p.A += z * p.batch_a;
        p.W += (z / p.batch_w_div) * p.batch_w;
        if (p.out16) p.out16 += z * p.batch_o16;
        if (p.out32) p.out32 += z * p.batch_o32;
    }
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // Workgroup -> tile: XCD x (= id % 8) takes a contiguous range of tiles in
    // a grouped order (kGroup row panels, column by column), so the tiles an
    // XCD runs together form a compact block whose A and W panels stay in its L2.
    const int ntn = (p.N + BN - 1) / BN;
    const int ntm = (p.M + BM - 1) / BM;
    const int nwg = ntn * ntm;
    const int id = blockIdx.x;
    const int per = nwg / 8;
    const int order = (id < per * 8) ? (id % 8) * per + id / 8 : id;
    constexpr int kGroup = 8;
    const int gsz = kGroup * ntn;
    const int grp = order / gsz, gm = min(kGroup, ntm - grp * kGroup);
    const int within = order - grp * gsz;
    const int tm = grp * kGroup + within % gm, tn = within / gm;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;

    // Per-lane global source of each wave load (row clamped into range; the
    // rows past M / N are computed but never stored).
    const int lrow = lane >> 3;
    // chunk fetched by this lane for 8-row block blk (rows 8 blk .. 8 blk + 7)
    auto lchunk = [&](int blk) { return (lane & 7) ^ ((4 * (blk & 1) + (lrow >> 1)) & 7); };
    const f16 * asrc[G::A_LOADS];
    const f16 * bsrc[G::B_LOADS];
    // conv: output pixel (image, y, x) of each A load row; asrc is the image's bordered input base
    int cy[CONV ? G::A_LOADS : 1], cx[CONV ? G::A_LOADS : 1];
#pragma unroll
    for (int i = 0; i < G::A_LOADS; ++i) {
        const int r = (wid + i * G::NW) * 8 + lrow;
        const int m = min(m0 + r, p.M - 1);
        if constexpr (CONV == 0) {
            asrc[i] = reinterpret_cast<const f16 *>(p.A) + (int64_t)m * p.lda + lchunk(wid + i * G::NW) * 8;
        } else {
            const int hw = p.conv_h * p.conv_w;
            const int img = m / hw, rem = m - img * hw;
            cy[i] = rem / p.conv_w;
            cx[i] = rem - cy[i] * p.conv_w;
            const int ih = CONV == 2 ? p.conv_h / 2 : p.conv_h, iw = CONV == 2 ? p.conv_w / 2 : p.conv_w;
            asrc[i] = reinterpret_cast<const f16 *>(p.A) + (int64_t)img * (ih + 2) * (iw + 2) * p.lda +
                      lchunk(wid + i * G::NW) * 8;
        }
    }
#pragma unroll
    for (int i = 0; i < G::B_LOADS; ++i) {
        const int r = (wid + i * G::NW) * 8 + lrow;
        bsrc[i] = reinterpret_cast<const f16 *>(p.W) + (int64_t)min(n0 + r, p.N - 1) * p.ldw + lchunk(wid + i * G::NW) * 8;
    }
    auto issue = [&](int kt, int st) {
        unsigned char * base = smem + st * G::STAGE_BYTES;
        const int k0 = kt * kBK;
        if constexpr (CONV == 0) {
#pragma unroll
            for (int i = 0; i < G::A_LOADS; ++i)
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(asrc[i] + k0),
                                                 SANA_LDS(base + (wid + i * G::NW) * 1024), 16, 0, 0);
        } else {
            // k-tile kt = (tap, 64-channel chunk): one 128-byte run of the source pixel
            const int cpt = (int)(p.lda >> 6);
            const int tap = kt / cpt, c0 = (kt - tap * cpt) << 6;
            const int ky = tap / 3, kx = tap - 3 * ky;
#pragma unroll
            for (int i = 0; i < G::A_LOADS; ++i) {
                int sr, sc, wp;
                if constexpr (CONV == 1) {
                    // bordered input: output (y, x) at tap (ky, kx) reads (y + ky, x + kx)
                    sr = cy[i] + ky;
                    sc = cx[i] + kx;
                    wp = p.conv_w + 2;
                } else {
                    // upsampled coordinate u = y + ky - 1 in [-1, conv_h]: the border outside
                    const int u = cy[i] + ky - 1, v = cx[i] + kx - 1;
                    sr = u < 0 ? 0 : (u >= p.conv_h ? p.conv_h / 2 + 1 : (u >> 1) + 1);
                    sc = v < 0 ? 0 : (v >= p.conv_w ? p.conv_w / 2 + 1 : (v >> 1) + 1);
                    wp = p.conv_w / 2 + 2;
                }
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(asrc[i] + ((int64_t)sr * wp + sc) * p.lda + c0),
                                                 SANA_LDS(base + (wid + i * G::NW) * 1024), 16, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < G::B_LOADS; ++i)
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(bsrc[i] + k0), SANA_LDS(base + G::A_BYTES + (wid + i * G::NW) * 1024),
                                             16, 0, 0);
    };

    f32x16 acc[G::TM][G::TN];
#pragma unroll
    for (int i = 0; i < G::TM; ++i)
#pragma unroll
        for (int j = 0; j < G::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Operand read offsets within a stage: row R, chunk ch -> R*128 + ((ch ^ ((R >> 1) & 7)) << 4).
    const int arow0 = wm * G::WTM + (lane & 31);
    const int brow0 = wn * G::WTN + (lane & 31);
    const int khalf = lane >> 5;

    // Operand fragments are double-buffered in registers: the LDS reads of
    // k-step s+1 are in flight while the MFMAs of step s run.  The tile
    // boundary (wait for the next tile's DMA, barrier, refill the freed stage)
    // is placed after the last step's MFMAs are issued, so it overlaps them.
    constexpr int NS = kBK / 16;               // MFMA k-steps per tile
    constexpr int NB = (SCHED == 1 || SCHED == 3) ? NS : 2;    // fragment buffers
    f16x8 af[NB][G::TM], bf[NB][G::TN];
    auto load_frags = [&](int stage, int s, int buf) {
        const unsigned char * sa = smem + stage * G::STAGE_BYTES;
        const unsigned char * sb = sa + G::A_BYTES;
        const int ch = 2 * s + khalf;
#pragma unroll
        for (int i = 0; i < G::TM; ++i) {
            const int R = arow0 + i * 32;
            af[buf][i] = *reinterpret_cast<const f16x8 *>(sa + R * 128 + ((ch ^ ((R >> 1) & 7)) << 4));
        }
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
            const int R = brow0 + j * 32;
            bf[buf][j] = *reinterpret_cast<const f16x8 *>(sb + R * 128 + ((ch ^ ((R >> 1) & 7)) << 4));
        }
    };
    // The MFMA computes the transposed tile, D^T = W_frag * A_frag^T, so that
    // lane l of wave tile (i, j) holds output row wm*WTM + i*32 + (l & 31) and,
    // in acc[i][j][4g .. 4g+3], the four consecutive columns
    // wn*WTN + j*32 + 8g + 4(l >> 5) + 0..3: the epilogue then writes 16-byte
    // (fp32) or 8-byte (fp16) row runs to LDS instead of single elements.
    auto mfmas = [&](int buf) {
#pragma unroll
        for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int j = 0; j < G::TN; ++j) acc[i][j] = mfma_32x32x16(bf[buf][j], af[buf][i], acc[i][j]);
    };

    // Residual epilogue inputs (x rows and the gate), loaded before the main loop
    // so their latency hides behind it: single-pass epilogues with at most two
    // rows per thread (the 64 x 64 and 128 x 64 tiles), plain A.  The thread ->
    // (8-column chunk, rows) map is the epilogue's.
    constexpr int ECPR = BN / 8, ERSTEP = G::NT / ECPR, ERPT = (G::EPI_ROWS + ERSTEP - 1) / ERSTEP;
    constexpr bool kPrefetch = MODE == kGemmResidual && CONV == 0 && G::EPI_ROWS == BM && ERPT <= 2;
    float xpre[kPrefetch ? ERPT : 1][8], gpre[kPrefetch ? ERPT : 1][8], bpre[8];
    // The fp16 epilogue's bias, one column per lane and wave sub-tile (column
    // wn*WTN + j*32 + (lane & 31)); the epilogue hands each lane the values of
    // its 4-column runs with lane shuffles.  Loaded here, its latency hides
    // behind the main loop (loaded in the epilogue it cost 1-2 us per launch).
    constexpr bool kH16 = MODE == kGemmQKV || (MODE == kGemmStore && ACT != kActGeglu);
    float bcol[kH16 ? G::TN : 1];
    if constexpr (kH16) {
#pragma unroll
        for (int j = 0; j < G::TN; ++j) {
            const int c = n0 + wn * G::WTN + j * 32 + (lane & 31);
            bcol[j] = (p.bias && c < p.N) ? p.bias[c] : 0.0f;
        }
    }
    if constexpr (kPrefetch) {
        const int col = n0 + (tid % ECPR) * 8;
        const int nc = min(8, p.N - col);
        const bool act = nc > 0 && tid < ERSTEP * ECPR;
        // bias of the thread's 8 columns
#pragma unroll
        for (int e = 0; e < 8; ++e) bpre[e] = 0.0f;
        if (act && p.bias) {
            if (p.vec && nc == 8) {
                const float4 b0 = *reinterpret_cast<const float4 *>(p.bias + col);
                const float4 b1 = *reinterpret_cast<const float4 *>(p.bias + col + 4);
                bpre[0] = b0.x; bpre[1] = b0.y; bpre[2] = b0.z; bpre[3] = b0.w;
                bpre[4] = b1.x; bpre[5] = b1.y; bpre[6] = b1.z; bpre[7] = b1.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (e < nc) bpre[e] = p.bias[col + e];
            }
        }
#pragma unroll
        for (int k = 0; k < ERPT; ++k) {
            const int row = m0 + tid / ECPR + k * ERSTEP;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xpre[k][e] = 0.0f;
                gpre[k][e] = 1.0f;
            }
            if (!act || row >= p.M) continue;
            const float * xr = p.out32 + (int64_t)row * p.ldo32 + col;
            const float * ga = p.gate_a ? p.gate_a + (int64_t)(row / p.rows_per_batch) * p.gate_stride + col : nullptr;
            if (p.vec && nc == 8) {
                const float4 x0 = *reinterpret_cast<const float4 *>(xr);
                const float4 x1 = *reinterpret_cast<const float4 *>(xr + 4);
                xpre[k][0] = x0.x; xpre[k][1] = x0.y; xpre[k][2] = x0.z; xpre[k][3] = x0.w;
                xpre[k][4] = x1.x; xpre[k][5] = x1.y; xpre[k][6] = x1.z; xpre[k][7] = x1.w;
                if (ga) {
                    const float4 g0 = *reinterpret_cast<const float4 *>(ga);
                    const float4 g1 = *reinterpret_cast<const float4 *>(ga + 4);
                    gpre[k][0] = g0.x; gpre[k][1] = g0.y; gpre[k][2] = g0.z; gpre[k][3] = g0.w;
                    gpre[k][4] = g1.x; gpre[k][5] = g1.y; gpre[k][6] = g1.z; gpre[k][7] = g1.w;
                    if (p.gate_t) {
                        const float4 t0 = *reinterpret_cast<const float4 *>(p.gate_t + col);
                        const float4 t1 = *reinterpret_cast<const float4 *>(p.gate_t + col + 4);
                        gpre[k][0] += t0.x; gpre[k][1] += t0.y; gpre[k][2] += t0.z; gpre[k][3] += t0.w;
                        gpre[k][4] += t1.x; gpre[k][5] += t1.y; gpre[k][6] += t1.z; gpre[k][7] += t1.w;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (e >= nc) continue;
                    xpre[k][e] = xr[e];
                    if (ga) gpre[k][e] = ga[e] + (p.gate_t ? p.gate_t[col + e] : 0.0f);
                }
            }
        }
    }

    const int KT = p.K / kBK;
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
        if (s < KT) issue(s, s);
    wait_stages<G::LOADS, STAGES>(min(STAGES - 1, KT - 1));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (SCHED == 3) {
        // Early stage release: all fragments of tile kt are read into registers,
        // a barrier confirms every wave is done with the stage, and the stage is
        // refilled with tile kt+STAGES before the tile's MFMAs run.  With two
        // stages, two tiles of DMA are in flight during the MFMAs instead of one,
        // which hides the longer latency of weights that come from HBM.
        for (int kt = 0; kt < KT; ++kt) {
            const int st = kt % STAGES;
            if (kt > 0) {
                __builtin_amdgcn_sched_barrier(0);
                wait_stages<G::LOADS, STAGES>(min(STAGES - 1, KT - 1 - kt));
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int s = 0; s < NS; ++s) load_frags(st, s, s);
            __builtin_amdgcn_sched_barrier(0);
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if (kt + STAGES < KT) issue(kt + STAGES, st);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < NS; ++s) mfmas(s);
        }
    } else if constexpr (SCHED == 1) {
        // every fragment of the tile is requested right after the barrier; the
        // MFMAs of step s wait only for the reads of steps <= s (in-order lgkmcnt)
        for (int kt = 0; kt < KT; ++kt) {
            const int st = kt % STAGES;
#pragma unroll
            for (int s = 0; s < NS; ++s) load_frags(st, s, s);
#pragma unroll
            for (int s = 0; s < NS; ++s) mfmas(s);
            if (kt + 1 < KT) {
                __builtin_amdgcn_sched_barrier(0);
                wait_stages<G::LOADS, STAGES>(min(STAGES - 2, KT - 2 - kt));
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (kt + STAGES < KT) issue(kt + STAGES, st);
            }
        }
    } else {
        // Operand fragments double-buffered in registers: the LDS reads of
        // k-step s+1 are in flight while the MFMAs of step s run.  The tile
        // boundary (wait for the next tile's DMA, barrier, refill the freed
        // stage) follows the last step's MFMAs, so it overlaps them.
        load_frags(0, 0, 0);
        for (int kt = 0; kt < KT; ++kt) {
            const int st = kt % STAGES;
#pragma unroll
            for (int s = 0; s < NS - 1; ++s) {
                load_frags(st, s + 1, (s + 1) & 1);
                mfmas(s & 1);
                if constexpr (SCHED == 2) {
                    __builtin_amdgcn_sched_group_barrier(0x100, G::TM + G::TN, 0);  // DS reads of step s+1
                    __builtin_amdgcn_sched_group_barrier(0x008, G::TM * G::TN, 0);  // then MFMAs of step s
                }
            }
            mfmas((NS - 1) & 1);
            if (kt + 1 < KT) {
                __builtin_amdgcn_sched_barrier(0);
                // tile kt+1 has landed (this wave's DMA), then every wave's has and
                // every wave is done reading stage st, which takes tile kt+STAGES.
                wait_stages<G::LOADS, STAGES>(min(STAGES - 2, KT - 2 - kt));
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (kt + STAGES < KT) issue(kt + STAGES, st);
                load_frags((kt + 1) % STAGES, 0, 0);
            }
        }
    }

    // ------------------------------------------------------------ epilogue
    // fp16 output row of tile row `row`: plain, or inside the bordered grid of a conv output
    auto orow16 = [&](int row) -> int64_t {
        if constexpr (CONV != 0) {
            if (p.out16_pad) {
                const int hw = p.conv_h * p.conv_w;
                const int img = row / hw, rem = row - img * hw;
                const int y = rem / p.conv_w, x = rem - y * p.conv_w;
                return ((int64_t)img * (p.conv_h + 2) + y + 1) * (p.conv_w + 2) + x + 1;
            }
        }
        return row;
    };
    // fp16-only outputs (plain stores with no fp32 copy, and the q|k|v split):
    // bias, activation and the fp16 rounding are applied to the accumulators in
    // registers (the same operations, in the same order, as the fp32-staged
    // path below), the rounded tile is staged in LDS once as fp16 (8-byte row
    // runs, rows 16-byte aligned), and every thread then issues all of its
    // 16-byte LDS reads before its 16-byte global stores.  Against the fp32
    // staging this halves the LDS bytes, needs a single pass for every tile
    // shape, and keeps several stores in flight per thread.
    if constexpr (MODE == kGemmQKV || (MODE == kGemmStore && ACT != kActGeglu)) {
        if (p.vec && !p.out32) {
            constexpr int LDH = BN + 8;
            static_assert(BM * LDH * 2 <= G::LDS_BYTES, "fp16 epilogue tile");
            f16 * ht = reinterpret_cast<f16 *>(smem);
            __syncthreads();  // every wave is done reading the operand ring
#pragma unroll
            for (int j = 0; j < G::TN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = wn * G::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
                    const int col = n0 + c;
                    float b4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) b4[e] = __shfl(bcol[j], 8 * g + 4 * (lane >> 5) + e, 64);
                    // q and k sections are ReLU'd (a 4-column run never straddles
                    // a section: qkv_c is a multiple of 8)
                    const bool relu = MODE == kGemmQKV && col < 2 * p.qkv_c;
#pragma unroll
                    for (int i = 0; i < G::TM; ++i) {
                        const int row = wm * G::WTM + i * 32 + (lane & 31);
                        f16x4 h;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float v = acc[i][j][4 * g + e] + b4[e];
                            if constexpr (ACT == kActSilu) v = silu_fast(v);
                            if constexpr (ACT == kActGelu) v = gelu_tanh_f(v);
                            if (relu) v = fmaxf(v, 0.0f);
                            h[e] = (f16)v;
                        }
                        *reinterpret_cast<f16x4 *>(ht + row * LDH + c) = h;
                    }
                }
            __syncthreads();
            // row-major stores (the whole tile, or the q section of the split)
            constexpr int HCPR = BN / 8, CHUNKS = BM * HCPR;
            constexpr int PER = (CHUNKS + G::NT - 1) / G::NT;
            f16x8 hv[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int idx = tid + k * G::NT;
                if (CHUNKS % G::NT == 0 || idx < CHUNKS)
                    hv[k] = *reinterpret_cast<const f16x8 *>(ht + (idx / HCPR) * LDH + (idx % HCPR) * 8);
            }
            f16 * o16 = reinterpret_cast<f16 *>(p.out16);
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int idx = tid + k * G::NT;
                if (CHUNKS % G::NT != 0 && idx >= CHUNKS) continue;
                const int row = m0 + idx / HCPR, col = n0 + (idx % HCPR) * 8;
                if (row >= p.M || col >= p.N) continue;
                if constexpr (MODE == kGemmQKV) {
                    if (col >= p.qkv_c) continue;
                }
                f16 * dst = o16 + orow16(row) * p.ldo16 + col;
                if (col + 8 <= p.N) {
                    *reinterpret_cast<f16x8 *>(dst) = hv[k];
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (col + e < p.N) dst[e] = hv[k][e];
                }
            }
            if constexpr (MODE == kGemmQKV) {
                // k and v sections: items (column, 8-row octet), 32 consecutive
                // columns of one octet per 32 items; each item leaves as one
                // 16-byte token run of relu(K)^T or V^T.  Rows of an octet share
                // a batch (qkv_n % 8 == 0).
                constexpr int OCT = BM / 8;
                const int C3 = p.qkv_c;
                for (int item = tid; item < BN * OCT; item += G::NT) {
                    const int c32 = item % 32, rest = item / 32;
                    const int oct = rest % OCT, cl = (rest / OCT) * 32 + c32;
                    const int col = n0 + cl, row0 = m0 + oct * 8;
                    if (col >= p.N || row0 >= p.M || col < C3) continue;
                    const bool is_k = col < 2 * C3;
                    const int ch = col - (is_k ? C3 : 2 * C3);
                    f16x8 h;
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) h[jj] = ht[(oct * 8 + jj) * LDH + cl];
                    const int b = row0 / p.qkv_n, t0 = row0 - b * p.qkv_n;
                    f16 * dst = reinterpret_cast<f16 *>(is_k ? p.kt16 : p.vt16);
                    *reinterpret_cast<f16x8 *>(dst + ((int64_t)b * C3 + ch) * p.qkv_n + t0) = h;
                }
            }
            return;
        }
    }
    {
        float * ct = reinterpret_cast<float *>(smem);
        constexpr int LDC = BN + G::CPAD;
        constexpr int ER = G::EPI_ROWS;  // tile rows staged per pass
        // Each thread owns one 8-column chunk of the tile for all its rows, so
        // the bias is fetched once; rows step by NT / CPR (threads past the
        // last whole row of chunks stay idle).
        constexpr int CPR = BN / 8;
        static_assert(G::NT >= CPR, "epilogue chunk mapping");
        const int c8 = (tid % CPR) * 8;
        const int col = n0 + c8;
        const int nc = min(8, p.N - col);
        bool active = nc > 0 && tid < (G::NT / CPR) * CPR;
        if constexpr (MODE == kGemmQKV) active = active && col < p.qkv_c;  // k / v columns: item loop
        const bool vec8 = p.vec && nc == 8;
        float bv[8];
        if constexpr (kPrefetch) {
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = bpre[e];
        } else if (!active) {
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = 0.0f;
        } else if (MODE == kGemmVT) {  // bias per row, added below
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = 0.0f;
        } else if (p.bias && vec8) {
            const float4 b0 = *reinterpret_cast<const float4 *>(p.bias + col);
            const float4 b1 = *reinterpret_cast<const float4 *>(p.bias + col + 4);
            bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w;
            bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) bv[e] = (p.bias && e < nc) ? p.bias[col + e] : 0.0f;
        }
        for (int pass = 0; pass < BM / ER; ++pass) {
            __syncthreads();  // the operand ring (pass 0) or the previous pass's rows are free
            if (ER == BM || wm == pass) {
                // 16-byte row runs (rows are 16-byte aligned: LDC = BN + 4, BN a multiple of 8)
#pragma unroll
                for (int i = 0; i < G::TM; ++i)
#pragma unroll
                    for (int j = 0; j < G::TN; ++j) {
                        const int rr = (wm * G::WTM - pass * ER) + i * 32 + (lane & 31);
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int c = wn * G::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
                            *reinterpret_cast<float4 *>(&ct[rr * LDC + c]) =
                                make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                        }
                    }
            }
            __syncthreads();
            if constexpr (MODE == kGemmQKV) {
                // k and v sections: items (column, 8-row octet).  32 consecutive
                // items take 32 consecutive columns of one octet and the next 32 the
                // same columns one octet further: rows 8 apart are 32 banks apart
                // (LDC = BN + 4), so a wave's fp32 LDS reads hit 64 distinct banks,
                // and each column's two octets leave as one 32-byte token run.  Rows
                // of an octet share a batch (qkv_n % 8 == 0).  The q section is
                // handled below as a plain store.
                constexpr int OCT = ER / 8;
                static_assert(BN % 32 == 0, "32-column item groups");
                const int C3 = p.qkv_c;
                for (int item = tid; item < BN * OCT; item += G::NT) {
                    const int c32 = item % 32, rest = item / 32;
                    const int oct = rest % OCT, cl = (rest / OCT) * 32 + c32;
                    const int col = n0 + cl, row0 = m0 + pass * ER + oct * 8;
                    if (col >= p.N || row0 >= p.M || col < C3) continue;
                    const bool is_k = col < 2 * C3;
                    const int ch = col - (is_k ? C3 : 2 * C3);
                    const float bcol = p.bias ? p.bias[col] : 0.0f;
                    f16x8 h;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        float v = ct[(oct * 8 + j) * LDC + cl] + bcol;
                        if (is_k) v = fmaxf(v, 0.0f);
                        h[j] = (f16)v;
                    }
                    const int b = row0 / p.qkv_n, t0 = row0 - b * p.qkv_n;
                    f16 * dst = reinterpret_cast<f16 *>(is_k ? p.kt16 : p.vt16);
                    *reinterpret_cast<f16x8 *>(dst + ((int64_t)b * C3 + ch) * p.qkv_n + t0) = h;
                }
            }
            if constexpr (MODE == kGemmVT) {
                // element (m, n), m = blk * vt_rows + r, n = b * vt_cols + j, goes to
                // out16[((blk * vt_batch + b) * vt_rows + r) * vt_ld + j]; bias per row.
                // A chunk inside one batch's columns leaves as two 8-byte stores
                // (vt_cols need not be a multiple of 8, so j is a multiple of 4 at best).
                const int vb = col / p.vt_cols, vj = col - vb * p.vt_cols;
                const bool vec4 = p.vec && nc == 8 && vj + 8 <= p.vt_cols && (vj & 3) == 0 && (p.vt_ld & 3) == 0;
                f16 * o16 = reinterpret_cast<f16 *>(p.out16);
                if (active) {
                    for (int rr = tid / CPR; rr < ER; rr += G::NT / CPR) {
                        const int row = m0 + pass * ER + rr;
                        if (row >= p.M) break;
                        const int blk = row / p.vt_rows, r = row - blk * p.vt_rows;
                        const float bvr = p.bias ? p.bias[row] : 0.0f;
                        const float4 v0 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8]);
                        const float4 v1 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8 + 4]);
                        const float v[8] = {v0.x + bvr, v0.y + bvr, v0.z + bvr, v0.w + bvr,
                                            v1.x + bvr, v1.y + bvr, v1.z + bvr, v1.w + bvr};
                        if (vec4) {
                            f16 * dst = o16 + ((int64_t)(blk * p.vt_batch + vb) * p.vt_rows + r) * p.vt_ld + vj;
                            f16x4 h0, h1;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                h0[e] = (f16)v[e];
                                h1[e] = (f16)v[4 + e];
                            }
                            *reinterpret_cast<f16x4 *>(dst) = h0;
                            *reinterpret_cast<f16x4 *>(dst + 4) = h1;
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                if (e >= nc) continue;
                                const int b = (col + e) / p.vt_cols, jj = col + e - b * p.vt_cols;
                                o16[((int64_t)(blk * p.vt_batch + b) * p.vt_rows + r) * p.vt_ld + jj] = (f16)v[e];
                            }
                        }
                    }
                }
            } else if (active && MODE != kGemmResidual) {
                for (int rr = tid / CPR; rr < ER; rr += G::NT / CPR) {
                    const int row = m0 + pass * ER + rr;
                    if (row >= p.M) break;
                    const float4 v0 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8]);
                    const float4 v1 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8 + 4]);
                    float v[8] = {v0.x + bv[0], v0.y + bv[1], v0.z + bv[2], v0.w + bv[3],
                                  v1.x + bv[4], v1.y + bv[5], v1.z + bv[6], v1.w + bv[7]};
                    if constexpr (MODE == kGemmStore && ACT == kActGeglu) {
                        // gate / up column pairs -> 4 gated outputs at column col / 2
                        f16x4 h;
#pragma unroll
                        for (int e = 0; e < 4; ++e) h[e] = (f16)(gelu_tanh_f(v[2 * e]) * v[2 * e + 1]);
                        f16 * o = reinterpret_cast<f16 *>(p.out16) + (int64_t)row * p.ldo16 + col / 2;
                        if (vec8) {
                            *reinterpret_cast<f16x4 *>(o) = h;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (2 * e + 1 < nc) o[e] = h[e];
                        }
                    } else if constexpr (MODE == kGemmStore || MODE == kGemmQKV) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if constexpr (ACT == kActSilu) v[e] = silu_fast(v[e]);
                            if constexpr (ACT == kActGelu) v[e] = gelu_tanh_f(v[e]);
                            if constexpr (MODE == kGemmQKV) v[e] = fmaxf(v[e], 0.0f);
                        }
                        if (vec8) {
                            if (p.out16) {
                                f16x8 h;
#pragma unroll
                                for (int e = 0; e < 8; ++e) h[e] = (f16)v[e];
                                *reinterpret_cast<f16x8 *>(reinterpret_cast<f16 *>(p.out16) + orow16(row) * p.ldo16 + col) = h;
                            }
                            if (p.out32) {
                                float * o = p.out32 + (int64_t)row * p.ldo32 + col;
                                *reinterpret_cast<float4 *>(o) = make_float4(v[0], v[1], v[2], v[3]);
                                *reinterpret_cast<float4 *>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
                            }
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e) {  // static indices: v stays in registers
                                if (e >= nc) continue;
                                if (p.out16) reinterpret_cast<f16 *>(p.out16)[orow16(row) * p.ldo16 + col + e] = (f16)v[e];
                                if (p.out32) p.out32[(int64_t)row * p.ldo32 + col + e] = v[e];
                            }
                        }
                    }
                }
            }
            if constexpr (MODE == kGemmResidual) {
                if (active) {
                    // x += gate * (acc + bias).  All of this
                    // thread's residual rows are loaded first (one batch of loads in
                    // flight), then updated and stored.
                    constexpr int RSTEP = G::NT / CPR;
                    constexpr int RPT = (ER + RSTEP - 1) / RSTEP;
                    const int rbase = tid / CPR;
                    float xin[RPT][8];
#pragma unroll
                    for (int k = 0; k < RPT; ++k) {
                        const int rr = rbase + k * RSTEP;
                        const int row = m0 + pass * ER + rr;
#pragma unroll
                        for (int e = 0; e < 8; ++e) xin[k][e] = 0.0f;
                        if constexpr (kPrefetch) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) xin[k][e] = xpre[k][e];
                            continue;
                        }
                        if (rr >= ER || row >= p.M) continue;
                        bool gathered = false;
                        if constexpr (CONV == 2) {
                            if (p.up_src) {
                                // the residual starts as the pixel-shuffled channel-repeat
                                // shortcut of the low-resolution input
                                const int hw = p.conv_h * p.conv_w;
                                const int img = row / hw, rem = row - img * hw;
                                const int Y = rem / p.conv_w, X = rem - Y * p.conv_w;
                                const float * src =
                                    p.up_src + ((int64_t)(img * (p.conv_h / 2) + (Y >> 1)) * (p.conv_w / 2) + (X >> 1)) *
                                                   p.up_c;
                                const int q = 2 * (Y & 1) + (X & 1);
#pragma unroll
                                for (int e = 0; e < 8; ++e)
                                    if (e < nc) xin[k][e] = src[((col + e) * 4 + q) / p.up_rep];
                                gathered = true;
                            }
                        }
                        if (!gathered) {
                            const float * xr = p.out32 + (int64_t)row * p.ldo32 + col;
                            if (vec8) {
                                const float4 x0 = *reinterpret_cast<const float4 *>(xr);
                                const float4 x1 = *reinterpret_cast<const float4 *>(xr + 4);
                                xin[k][0] = x0.x; xin[k][1] = x0.y; xin[k][2] = x0.z; xin[k][3] = x0.w;
                                xin[k][4] = x1.x; xin[k][5] = x1.y; xin[k][6] = x1.z; xin[k][7] = x1.w;
                            } else {
#pragma unroll
                                for (int e = 0; e < 8; ++e)
                                    if (e < nc) xin[k][e] = xr[e];
                            }
                        }
                    }
#pragma unroll
                    for (int k = 0; k < RPT; ++k) {
                        const int rr = rbase + k * RSTEP;
                        const int row = m0 + pass * ER + rr;
                        if (rr >= ER || row >= p.M) continue;
                        const float4 v0 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8]);
                        const float4 v1 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8 + 4]);
                        float v[8] = {v0.x + bv[0], v0.y + bv[1], v0.z + bv[2], v0.w + bv[3],
                                      v1.x + bv[4], v1.y + bv[5], v1.z + bv[6], v1.w + bv[7]};
                        const int b = row / p.rows_per_batch;
                        float g[8];
                        if constexpr (kPrefetch) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) g[e] = gpre[k][e];
                        } else if (p.gate_a && vec8) {
                            const float * ga = p.gate_a + (int64_t)b * p.gate_stride + col;
                            const float4 g0 = *reinterpret_cast<const float4 *>(ga);
                            const float4 g1 = *reinterpret_cast<const float4 *>(ga + 4);
                            g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;
                            g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
                            if (p.gate_t) {
                                const float4 t0 = *reinterpret_cast<const float4 *>(p.gate_t + col);
                                const float4 t1 = *reinterpret_cast<const float4 *>(p.gate_t + col + 4);
                                g[0] += t0.x; g[1] += t0.y; g[2] += t0.z; g[3] += t0.w;
                                g[4] += t1.x; g[5] += t1.y; g[6] += t1.z; g[7] += t1.w;
                            }
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                g[e] = 1.0f;
                                if (p.gate_a && e < nc) {
                                    g[e] = p.gate_a[(int64_t)b * p.gate_stride + col + e];
                                    if (p.gate_t) g[e] += p.gate_t[col + e];
                                }
                            }
                        }
                        float x[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = xin[k][e] + g[e] * v[e];
                        float * xr = p.out32 + (int64_t)row * p.ldo32 + col;
                        if (vec8) {
                            *reinterpret_cast<float4 *>(xr) = make_float4(x[0], x[1], x[2], x[3]);
                            *reinterpret_cast<float4 *>(xr + 4) = make_float4(x[4], x[5], x[6], x[7]);
                            if (p.out16) {
                                f16x8 h;
#pragma unroll
                                for (int e = 0; e < 8; ++e) h[e] = (f16)x[e];
                                *reinterpret_cast<f16x8 *>(reinterpret_cast<f16 *>(p.out16) + orow16(row) * p.ldo16 + col) = h;
                            }
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                if (e >= nc) continue;
                                xr[e] = x[e];
                                if (p.out16) reinterpret_cast<f16 *>(p.out16)[orow16(row) * p.ldo16 + col + e] = (f16)x[e];
                            }
                        }
                    }
                }
            }
        }
    }
}

bool set_lds_limit(const void * k, size_t lds) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE, int SCHED, int ACT, int CONV = 0>
hipError_t launch_mode(const GemmParams & p, int tiles, hipStream_t s) {
    using G = Cfg<BM, BN, WM, WN, STAGES>;
    static const bool attr = set_lds_limit(
        reinterpret_cast<const void *>(&gemm_kernel<BM, BN, WM, WN, STAGES, MODE, SCHED, ACT, CONV>), G::LDS_BYTES);
    (void)attr;
    static const std::string name = "gemm_kernel<" + std::to_string(BM) + ", " + std::to_string(BN) + ", " +
                                    std::to_string(WM) + ", " + std::to_string(WN) + ", " + std::to_string(STAGES) +
                                    ", " + std::to_string(MODE) + ", " + std::to_string(SCHED) + ", " +
                                    std::to_string(ACT) + ", " + std::to_string(CONV) + ">";
    note_kernel(name.c_str());
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, STAGES, MODE, SCHED, ACT, CONV>), dim3(tiles, p.batch), dim3(G::NT),
                       G::LDS_BYTES, s, p);
    return hipGetLastError();
}

// Implicit 3x3 convolutions: plain stores (optionally SiLU) and residual updates.
template <int BM, int BN, int WM, int WN, int STAGES, int SCHED, int CONV>
hipError_t launch_conv_mode(const GemmParams & p, hipStream_t s) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    if (p.mode == kGemmResidual)
        return launch_mode<BM, BN, WM, WN, STAGES, kGemmResidual, SCHED, kActNone, CONV>(p, tiles, s);
    if (p.act == kActSilu) return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActSilu, CONV>(p, tiles, s);
    return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActNone, CONV>(p, tiles, s);
}

template <int BM, int BN, int WM, int WN, int STAGES, int SCHED>
hipError_t launch_conv(const GemmParams & p, hipStream_t s) {
    if (p.conv == 2) return launch_conv_mode<BM, BN, WM, WN, STAGES, SCHED, 2>(p, s);
    return launch_conv_mode<BM, BN, WM, WN, STAGES, SCHED, 1>(p, s);
}

template <int BM, int BN, int WM, int WN, int STAGES, int SCHED = 0>
hipError_t launch(const GemmParams & p, hipStream_t s) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    if (p.mode == kGemmResidual) return launch_mode<BM, BN, WM, WN, STAGES, kGemmResidual, SCHED, kActNone>(p, tiles, s);
    if (p.mode == kGemmVT) return launch_mode<BM, BN, WM, WN, STAGES, kGemmVT, SCHED, kActNone>(p, tiles, s);
    if (p.mode == kGemmQKV) return launch_mode<BM, BN, WM, WN, STAGES, kGemmQKV, SCHED, kActNone>(p, tiles, s);
    if (p.act == kActSilu) return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActSilu>(p, tiles, s);
    if (p.act == kActGelu) return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActGelu>(p, tiles, s);
    if (p.act == kActGeglu) return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActGeglu>(p, tiles, s);
    return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore, SCHED, kActNone>(p, tiles, s);
}

}  // namespace gemm_detail

using namespace gemm_detail;

hipError_t gemm(const GemmParams & p_in, hipStream_t s) {
    GemmParams p = p_in;
    if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % kBK != 0) return hipErrorInvalidValue;
    if (p.conv < 0 || p.conv > 2) return hipErrorInvalidValue;
    if (p.conv) {
        // implicit 3x3 conv: K = 9 taps x lda channels, M whole images of conv_h x conv_w
        if (p.conv_h <= 0 || p.conv_w <= 0 || p.lda <= 0 || p.lda % kBK || p.K != 9 * p.lda ||
            p.M % (p.conv_h * p.conv_w) || (p.mode != kGemmStore && p.mode != kGemmResidual) ||
            (p.conv == 2 && (p.conv_h % 2 || p.conv_w % 2)))
            return hipErrorInvalidValue;
    } else if (p.out16_pad || p.lda < p.K) {
        return hipErrorInvalidValue;
    }
    if (!p.A || !p.W || p.ldw < p.K || p.lda % 8 || p.ldw % 8) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.W)) & 15) return hipErrorInvalidValue;
    if (p.mode == kGemmResidual && !p.out32) return hipErrorInvalidValue;
    if (p.up_src && (p.conv != 2 || p.mode != kGemmResidual || p.up_c <= 0 || p.up_rep <= 0 ||
                     ((int64_t)p.N * 4 + p.up_rep - 1) / p.up_rep > p.up_c))
        return hipErrorInvalidValue;
    if (p.mode == kGemmVT && (!p.out16 || p.vt_rows <= 0 || p.vt_cols <= 0 || p.vt_batch <= 0 ||
                              p.vt_ld < p.vt_cols || p.N != p.vt_batch * p.vt_cols || p.M % p.vt_rows))
        return hipErrorInvalidValue;
    if (p.mode == kGemmStore && !p.out16 && !p.out32) return hipErrorInvalidValue;
    if (p.act < kActNone || p.act > kActGeglu) return hipErrorInvalidValue;
    if (p.act == kActGeglu && (p.mode != kGemmStore || p.conv || !p.out16 || p.out32 || p.N % 8 ||
                               p.ldo16 < p.N / 2 || p.batch != 1))
        return hipErrorInvalidValue;
    if (p.mode == kGemmQKV &&
        (!p.out16 || p.out32 || !p.kt16 || !p.vt16 || p.qkv_c <= 0 || p.qkv_c % 8 || p.N != 3 * p.qkv_c ||
         p.qkv_n <= 0 || p.qkv_n % 8 || p.M % p.qkv_n ||
         ((reinterpret_cast<uintptr_t>(p.kt16) | reinterpret_cast<uintptr_t>(p.vt16)) & 15)))
        return hipErrorInvalidValue;
    if (p.gate_a && p.rows_per_batch <= 0) return hipErrorInvalidValue;
    if (p.batch < 1 || p.batch > 65535 || p.batch_w_div < 1 ||
        (p.batch > 1 && (p.mode != kGemmStore || p.conv ||
                         ((p.batch_a | p.batch_w | p.batch_o16 | p.batch_o32) & 7) != 0)))
        return hipErrorInvalidValue;
    // 16-byte epilogue accesses need 8-element aligned rows and 16-byte aligned bases.
    bool vec = true;
    if (p.out16) vec = vec && p.ldo16 % 8 == 0 && (reinterpret_cast<uintptr_t>(p.out16) & 15) == 0;
    if (p.out32) vec = vec && p.ldo32 % 4 == 0 && (reinterpret_cast<uintptr_t>(p.out32) & 15) == 0;
    if (p.gate_a) vec = vec && p.gate_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(p.gate_a) & 15) == 0;
    if (p.gate_t) vec = vec && (reinterpret_cast<uintptr_t>(p.gate_t) & 15) == 0;
    if (p.bias) vec = vec && (reinterpret_cast<uintptr_t>(p.bias) & 15) == 0;
    p.vec = vec ? 1 : 0;
    if (p.conv) {
        // Early stage release is 2-6 % faster than schedule 1 on the VAE's
        // 3x3 convs (1024^2 x 128, 512^2 x 256, 256^2 x 512) but 15 % slower
        // on the upsampling convs, whose residual epilogue reads the shortcut.
        if (p.N <= 64) return launch_conv<128, 64, 2, 2, 2, 3>(p, s);
        if (p.conv == 2) return launch_conv<128, 128, 2, 2, 2, 1>(p, s);
        return launch_conv<128, 128, 2, 2, 2, 3>(p, s);
    }
    // Tile choice from sweeps on MI355X with cold weights (each GEMM's weights
    // come from HBM, as in the 28-block forward).  Every CU pulls at most
    // ~110 GB/s from L2, so larger tiles (fewer operand bytes per flop) win as
    // long as the grid still covers the 256 CUs:
    //  * grids of <= 160 128x128 tiles: shared with a concurrent launch (the
    //    two CFG branches), 64x64 tiles with three stages, early release for
    //    stores and the plain schedule for the residual GEMMs (1024 px forward
    //    5.055 -> 5.037 ms in one process);
    //    alone, 128x64 tiles with early stage release when that makes >= 256
    //    tiles, else 64x64 tiles (three stages and early release for K >= 2048:
    //    600-row caption projection, K = 2304: 20.3 -> 15.8 us);
    //  * grids of 161..256 128x128 tiles: 128x64 tiles with early release
    //    (738-row Gemma q|k|v 36.8 -> 31.3 us, its split output projection
    //    20.6 -> 17.2 us);
    //  * N a multiple of 192 and >= 768 128x192 tiles (1.5 rounds of the 512
    //    two-per-CU slots): 128x192, stores and residual alike (16384-row
    //    launches: 5-12 % faster than 128x128);
    //  * plain stores of N >= 3456 whose 128x192 grid fits one round of slots
    //    where the 128x128 grid does not: 128x192 (1024-row inverted FFN);
    //  * at most 5 row (or column) tiles of 128 against >= 128 of the other
    //    (the step's cross K 600 x 32256 and V^T 32256 x 600): 128x128 tiles
    //    of 8 waves (4 x 2, 32 x 64 per wave): 67.4 -> 60.0 us and 63.2 -> 60.8 us;
    //  * otherwise 128x128 tiles with two stages, two workgroups per CU.
    //  The QKV-split GEMM (both sizes) and, with 128x192 tiles, the residual
    //  GEMMs with K <= 1152 use workgroups of 8 waves (4 x 2): the forward at
    //  16384 rows per branch 54.00 -> 53.66 ms, at 1024 rows 5.089 -> 5.081 ms.
    // (tile counts are scaled by the launches that share the CUs, p.co, and
    // by the products of a batched launch)
    const int64_t co = std::max(p.co, 1) * (int64_t)p.batch;
    const int64_t tm128 = (p.M + 127) / 128;
    const int64_t t128 = tm128 * ((p.N + 127) / 128) * co;
    if (t128 <= 160) {
        if (co >= 2)
            return p.mode == kGemmResidual ? launch<64, 64, 2, 2, 3, 1>(p, s) : launch<64, 64, 2, 2, 3, 3>(p, s);
        if (tm128 * ((p.N + 63) / 64) >= 256) return launch<128, 64, 2, 2, 2, 3>(p, s);
        if (p.K >= 2048) return launch<64, 64, 2, 2, 3, 3>(p, s);
        return launch<64, 64, 2, 2, 2, 1>(p, s);
    }
    if (t128 <= 256 && tm128 * ((p.N + 63) / 64) * co >= 256) return launch<128, 64, 2, 2, 2, 3>(p, s);
    const int64_t tn128 = (p.N + 127) / 128;
    if (co == 1 && std::min(tm128, tn128) <= 5 && std::max(tm128, tn128) >= 128)
        return launch<128, 128, 4, 2, 2, 1>(p, s);
    const int64_t t192 = p.N % 192 == 0 ? tm128 * (p.N / 192) * co : 0;
    constexpr int64_t kSlots = 512;
    if (t192 >= kSlots * 3 / 2 ||
        (p.mode == kGemmStore && p.N >= 3456 && t192 > 0 && t192 <= kSlots && t128 > kSlots))
    {
        if (p.mode == kGemmQKV || (p.mode == kGemmResidual && p.K <= 1152)) return launch<128, 192, 4, 2, 2, 1>(p, s);
        return launch<128, 192, 2, 2, 2, 1>(p, s);
    }
    if (p.mode == kGemmQKV) return launch<128, 128, 4, 2, 2, 1>(p, s);
    return launch<128, 128, 2, 2, 2, 1>(p, s);
}

}  // namespace sana
