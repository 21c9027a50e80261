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
//   * A STAGES-deep ring of LDS k-tiles (BK = 64): tile kt+STAGES-1 is in flight
//     while tile kt is multiplied, so HBM latency is covered by STAGES-1 tiles
//     of MFMA work.  Completion is tracked with an explicit vmcnt wait (the
//     loads of later tiles stay outstanding) and one s_barrier per k-tile.
//   * LDS rows are 128 bytes; 16-byte chunk c of row r is stored in slot
//     c ^ (r & 7).  The DMA writes lane l to slot l & 7 of row l >> 3, so lane
//     l fetches chunk (l & 7) ^ (l >> 3); an MFMA operand read (8 consecutive
//     rows, one chunk) then touches 8 distinct slots: no bank conflicts.
//   * Epilogue staged through LDS: the wave tiles are written to LDS in row
//     order, then every thread moves 8 consecutive columns with 16-byte
//     global accesses.
//
// The workgroup -> tile map is XCD-aware: gfx950 deals workgroups round-robin
// to 8 XCDs (each with its own L2), so workgroup id i is mapped to tile
// (i % 8) * (T / 8) + i / 8, giving each XCD a contiguous run of tiles in
// n-fastest order that shares A row panels in its L2.
//
// Fused epilogues (reference ops they replace):
//   store   : bias (+SiLU | +GELU-tanh), fp16 and/or fp32 out
//             (linear_3d_lastdim src/common_ops.cpp:177-209, silu src/tensor.cpp:551-555,
//              gelu_tanh src/transformer_ops.cpp:15-18)
//   residual: x += gate * (acc + bias), optional fp16 copy of the new x
//             (mul_inplace_broadcast_lastdim + add_inplace, src/tensor.cpp:101-160)
//   V^T     : transposed per-batch store of the cross-attention values.
#include <cstdlib>

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
    static constexpr int EPI_BYTES = BM * (BN + CPAD) * 4;
    static constexpr int LDS_BYTES = (STAGES * STAGE_BYTES > EPI_BYTES) ? STAGES * STAGE_BYTES : EPI_BYTES;
    static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "tile rows must split into 8-row wave loads");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
    static_assert(LOADS * (STAGES - 1) < 64, "vmcnt range");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");
};

// Wait until at most `keep` stages of this wave's loads are outstanding.
template <int LOADS, int STAGES>
SANA_DEV void wait_stages(int keep) {
    if constexpr (STAGES >= 4) {
        if (keep >= 2) { wait_vmcnt<2 * LOADS>(); return; }
    }
    if constexpr (STAGES >= 3) {
        if (keep >= 1) { wait_vmcnt<LOADS>(); return; }
    }
    wait_vmcnt<0>();
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmParams p) {
    using G = Cfg<BM, BN, WM, WN, STAGES>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int ntn = (p.N + BN - 1) / BN;
    const int ntm = (p.M + BM - 1) / BM;
    const int nwg = ntn * ntm;
    const int id = blockIdx.x;
    const int per = nwg / 8;
    const int tile = (id < per * 8) ? (id % 8) * per + id / 8 : id;
    const int tm = tile / ntn, tn = tile % ntn;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / WN, wn = wid % WN;

    // Per-lane global source of each wave load (row clamped into range; the
    // rows past M / N are computed but never stored).
    const int lrow = lane >> 3;
    const int lchunk = (lane & 7) ^ lrow;
    const f16 * asrc[G::A_LOADS];
    const f16 * bsrc[G::B_LOADS];
#pragma unroll
    for (int i = 0; i < G::A_LOADS; ++i) {
        const int r = (wid + i * G::NW) * 8 + lrow;
        asrc[i] = reinterpret_cast<const f16 *>(p.A) + (int64_t)min(m0 + r, p.M - 1) * p.lda + lchunk * 8;
    }
#pragma unroll
    for (int i = 0; i < G::B_LOADS; ++i) {
        const int r = (wid + i * G::NW) * 8 + lrow;
        bsrc[i] = reinterpret_cast<const f16 *>(p.W) + (int64_t)min(n0 + r, p.N - 1) * p.ldw + lchunk * 8;
    }
    auto issue = [&](int kt, int st) {
        unsigned char * base = smem + st * G::STAGE_BYTES;
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < G::A_LOADS; ++i)
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(asrc[i] + k0), SANA_LDS(base + (wid + i * G::NW) * 1024), 16, 0, 0);
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

    // Operand read offsets within a stage: row R, chunk ch -> R*128 + ((ch ^ (R & 7)) << 4).
    const int arow0 = wm * G::WTM + (lane & 31);
    const int brow0 = wn * G::WTN + (lane & 31);
    const int khalf = lane >> 5;

    const int KT = p.K / kBK;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < KT) issue(s, s);

    for (int kt = 0; kt < KT; ++kt) {
        // Tile kt has landed once at most min(STAGES-2, KT-1-kt) later stages are still in flight.
        wait_stages<G::LOADS, STAGES>(min(STAGES - 2, KT - 1 - kt));
        __builtin_amdgcn_s_barrier();
        if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        const unsigned char * sa = smem + (kt % STAGES) * G::STAGE_BYTES;
        const unsigned char * sb = sa + G::A_BYTES;
        // Operand fragments are double-buffered in registers: the reads of
        // k-step s+1 are issued before the MFMAs of step s.
        f16x8 af[2][G::TM], bf[2][G::TN];
        auto load_frags = [&](int s, int buf) {
            const int ch = 2 * s + khalf;
#pragma unroll
            for (int i = 0; i < G::TM; ++i) {
                const int R = arow0 + i * 32;
                af[buf][i] = *reinterpret_cast<const f16x8 *>(sa + R * 128 + ((ch ^ (R & 7)) << 4));
            }
#pragma unroll
            for (int j = 0; j < G::TN; ++j) {
                const int R = brow0 + j * 32;
                bf[buf][j] = *reinterpret_cast<const f16x8 *>(sb + R * 128 + ((ch ^ (R & 7)) << 4));
            }
        };
        load_frags(0, 0);
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            if (s + 1 < kBK / 16) load_frags(s + 1, (s + 1) & 1);
#pragma unroll
            for (int i = 0; i < G::TM; ++i)
#pragma unroll
                for (int j = 0; j < G::TN; ++j) acc[i][j] = mfma_32x32x16(af[s & 1][i], bf[s & 1][j], acc[i][j]);
        }
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (MODE == kGemmVT) {
        // Lane owns column (lane & 31) of each 32x32 block and rows
        // 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
        for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int j = 0; j < G::TN; ++j) {
                const int col = n0 + wn * G::WTN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * G::WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < p.M && col < p.N) {
                        float v = acc[i][j][r];
                        if (p.bias) v += p.bias[row];
                        const int blk = row / p.vt_rows, rr = row - blk * p.vt_rows;
                        const int b = col / p.vt_cols, jj = col - b * p.vt_cols;
                        reinterpret_cast<f16 *>(p.out16)[((int64_t)(blk * p.vt_batch + b) * p.vt_rows + rr) * p.vt_ld +
                                                         jj] = (f16)v;
                    }
                }
            }
        return;
    } else {
        __syncthreads();  // every wave is done reading the operand ring
        float * ct = reinterpret_cast<float *>(smem);
        constexpr int LDC = BN + G::CPAD;
#pragma unroll
        for (int i = 0; i < G::TM; ++i)
#pragma unroll
            for (int j = 0; j < G::TN; ++j) {
                const int c = wn * G::WTN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = wm * G::WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    ct[rr * LDC + c] = acc[i][j][r];
                }
            }
        __syncthreads();
        constexpr int CPR = BN / 8;  // 8-column chunks per row
        for (int q = tid; q < BM * CPR; q += G::NT) {
            const int rr = q / CPR, c8 = (q - rr * CPR) * 8;
            const int row = m0 + rr, col = n0 + c8;
            if (row >= p.M || col >= p.N) continue;
            const float4 v0 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8]);
            const float4 v1 = *reinterpret_cast<const float4 *>(&ct[rr * LDC + c8 + 4]);
            float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            const int nc = min(8, p.N - col);
            if (MODE == kGemmStore) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (p.bias && e < nc) v[e] += p.bias[col + e];
                    if (p.act == kActSilu) v[e] = silu_f(v[e]);
                    else if (p.act == kActGelu) v[e] = gelu_tanh_f(v[e]);
                }
                if (nc == 8 && p.vec) {
                    if (p.out16) {
                        f16x8 h;
#pragma unroll
                        for (int e = 0; e < 8; ++e) h[e] = (f16)v[e];
                        *reinterpret_cast<f16x8 *>(reinterpret_cast<f16 *>(p.out16) + (int64_t)row * p.ldo16 + col) = h;
                    }
                    if (p.out32) {
                        float * o = p.out32 + (int64_t)row * p.ldo32 + col;
                        *reinterpret_cast<float4 *>(o) = make_float4(v[0], v[1], v[2], v[3]);
                        *reinterpret_cast<float4 *>(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
                    }
                } else {
                    for (int e = 0; e < nc; ++e) {
                        if (p.out16) reinterpret_cast<f16 *>(p.out16)[(int64_t)row * p.ldo16 + col + e] = (f16)v[e];
                        if (p.out32) p.out32[(int64_t)row * p.ldo32 + col + e] = v[e];
                    }
                }
            } else {  // kGemmResidual: x += gate * (acc + bias)
                const int b = row / p.rows_per_batch;
                const float * ga = p.gate_a ? p.gate_a + (int64_t)b * p.gate_stride + col : nullptr;
                const float * gt = p.gate_t ? p.gate_t + col : nullptr;
                float * xr = p.out32 + (int64_t)row * p.ldo32 + col;
                if (nc == 8 && p.vec) {
                    float x[8], g[8];
                    const float4 x0 = *reinterpret_cast<const float4 *>(xr);
                    const float4 x1 = *reinterpret_cast<const float4 *>(xr + 4);
                    x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
                    x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        g[e] = ga ? ga[e] + (gt ? gt[e] : 0.0f) : 1.0f;
                        const float y = v[e] + (p.bias ? p.bias[col + e] : 0.0f);
                        x[e] = x[e] + g[e] * y;
                    }
                    *reinterpret_cast<float4 *>(xr) = make_float4(x[0], x[1], x[2], x[3]);
                    *reinterpret_cast<float4 *>(xr + 4) = make_float4(x[4], x[5], x[6], x[7]);
                    if (p.out16) {
                        f16x8 h;
#pragma unroll
                        for (int e = 0; e < 8; ++e) h[e] = (f16)x[e];
                        *reinterpret_cast<f16x8 *>(reinterpret_cast<f16 *>(p.out16) + (int64_t)row * p.ldo16 + col) = h;
                    }
                } else {
                    for (int e = 0; e < nc; ++e) {
                        const float g = ga ? ga[e] + (gt ? gt[e] : 0.0f) : 1.0f;
                        const float y = v[e] + (p.bias ? p.bias[col + e] : 0.0f);
                        const float nx = xr[e] + g * y;
                        xr[e] = nx;
                        if (p.out16) reinterpret_cast<f16 *>(p.out16)[(int64_t)row * p.ldo16 + col + e] = (f16)nx;
                    }
                }
            }
        }
    }
}

bool set_lds_limit(const void * k, size_t lds) {
    return hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
}

template <int BM, int BN, int WM, int WN, int STAGES, int MODE>
hipError_t launch_mode(const GemmParams & p, int tiles, hipStream_t s) {
    using G = Cfg<BM, BN, WM, WN, STAGES>;
    static const bool attr = set_lds_limit(reinterpret_cast<const void *>(&gemm_kernel<BM, BN, WM, WN, STAGES, MODE>),
                                           G::LDS_BYTES);
    (void)attr;
    hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, STAGES, MODE>), dim3(tiles), dim3(G::NT), G::LDS_BYTES, s, p);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch(const GemmParams & p, hipStream_t s) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    if (p.mode == kGemmResidual) return launch_mode<BM, BN, WM, WN, STAGES, kGemmResidual>(p, tiles, s);
    if (p.mode == kGemmVT) return launch_mode<BM, BN, WM, WN, STAGES, kGemmVT>(p, tiles, s);
    return launch_mode<BM, BN, WM, WN, STAGES, kGemmStore>(p, tiles, s);
}

}  // namespace gemm_detail

using namespace gemm_detail;

hipError_t gemm(const GemmParams & p_in, hipStream_t s) {
    GemmParams p = p_in;
    if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % kBK != 0) return hipErrorInvalidValue;
    if (!p.A || !p.W || p.lda < p.K || p.ldw < p.K || p.lda % 8 || p.ldw % 8) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.W)) & 15) return hipErrorInvalidValue;
    if (p.mode == kGemmResidual && !p.out32) return hipErrorInvalidValue;
    if (p.mode == kGemmVT && (!p.out16 || p.vt_rows <= 0 || p.vt_cols <= 0 || p.vt_batch <= 0 ||
                              p.vt_ld < p.vt_cols || p.N != p.vt_batch * p.vt_cols || p.M % p.vt_rows))
        return hipErrorInvalidValue;
    if (p.mode == kGemmStore && !p.out16 && !p.out32) return hipErrorInvalidValue;
    if (p.gate_a && p.rows_per_batch <= 0) return hipErrorInvalidValue;
    // 16-byte epilogue accesses need 8-element aligned rows and 16-byte aligned bases.
    bool vec = true;
    if (p.out16) vec = vec && p.ldo16 % 8 == 0 && (reinterpret_cast<uintptr_t>(p.out16) & 15) == 0;
    if (p.out32) vec = vec && p.ldo32 % 4 == 0 && (reinterpret_cast<uintptr_t>(p.out32) & 15) == 0;
    if (p.gate_a) vec = vec && p.gate_stride % 4 == 0;
    p.vec = vec ? 1 : 0;
    static const int forced = [] {
        const char * e = std::getenv("SANA_GEMM_VARIANT");
        return e ? std::atoi(e) : -1;
    }();
    switch (forced) {
        case 0: return launch<128, 128, 2, 2, 4>(p, s);
        case 1: return launch<128, 128, 2, 2, 3>(p, s);
        case 2: return launch<128, 128, 2, 2, 2>(p, s);
        case 3: return launch<128, 64, 2, 2, 4>(p, s);
        case 4: return launch<64, 64, 2, 2, 4>(p, s);
        case 5: return launch<256, 128, 2, 2, 3>(p, s);
        case 6: return launch<128, 256, 2, 2, 3>(p, s);
        case 7: return launch<64, 128, 2, 2, 4>(p, s);
        case 8: return launch<128, 64, 2, 2, 2>(p, s);
        case 9: return launch<64, 64, 2, 2, 2>(p, s);
        case 10: return launch<256, 128, 2, 2, 2>(p, s);
        case 11: return launch<128, 128, 1, 4, 3>(p, s);
        default: break;
    }
    // Tile choice from measured sweeps on MI355X: small grids (<= 160 tiles of
    // 128x128) need 64x64 tiles to occupy the 256 CUs; otherwise two-stage
    // 128-row tiles keep two workgroups resident per CU.
    const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
    if (t128 <= 160) return launch<64, 64, 2, 2, 2>(p, s);
    if (p.K >= 2048 || (t128 >= 300 && t128 <= 500) || t128 >= 2000) return launch<128, 128, 2, 2, 2>(p, s);
    return launch<128, 64, 2, 2, 2>(p, s);
}

}  // namespace sana
