// K1: MFMA GEMM for every dense projection of the DiT (QKV, attention output,
// cross-attention q/k/v/out, Mix-FFN inverted/point 1x1 convs, caption MLP).
//
// C[m, n] = sum_k A[m, k] * W[n, k], fp16 operands, fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  A (activations, token-major) and W (weights,
// PyTorch [out, in] order) are both K-contiguous, so each MFMA lane's operand
// (8 consecutive k of one row) is a single 16-byte LDS read.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, block tile BM x BN x 64,
// double-buffered LDS (global -> registers prefetch of tile k+1 overlaps the
// MFMAs of tile k; one barrier per k-tile).  LDS rows are 128 bytes; the 16-byte
// chunk c of row r is stored at chunk (c ^ (r & 7)) so that the 8 lanes of a
// ds_read_b128 phase hit 8 distinct chunk slots.
//
// The workgroup -> tile map is XCD-aware: gfx950 deals workgroups round-robin
// to 8 XCDs (each with its own L2), so workgroup id i is mapped to tile
// (i % 8) * (T / 8) + i / 8, giving each XCD a contiguous run of tiles in
// n-fastest order that shares one A row panel in its L2.
//
// Fused epilogues (reference ops they replace):
//   store  : bias (+SiLU | +GELU-tanh), fp16 and/or fp32 out
//            (linear_3d_lastdim src/common_ops.cpp:177-209, silu src/tensor.cpp:551-555,
//             gelu_tanh src/transformer_ops.cpp:15-18)
//   residual: x += gate * (acc + bias), optional fp16 copy of the new x
//            (mul_inplace_broadcast_lastdim + add_inplace, src/tensor.cpp:101-160)
//   V^T     : transposed per-batch store of the cross-attention values.
#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

constexpr int kBK = 64;

SANA_DEV int swz(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

template <int MODE>
SANA_DEV void epilogue(const GemmParams & p, int row, int col, float v) {
    if (MODE == kGemmVT) {
        if (p.bias) v += p.bias[row];
        const int blk = row / p.vt_rows, rr = row - blk * p.vt_rows;
        const int b = col / p.vt_cols, jj = col - b * p.vt_cols;
        reinterpret_cast<f16 *>(p.out16)[((int64_t)(blk * p.vt_batch + b) * p.vt_rows + rr) * p.vt_ld + jj] = (f16)v;
    } else if (MODE == kGemmResidual) {
        if (p.bias) v += p.bias[col];
        float g = 1.0f;
        if (p.gate_a) {
            const int b = row / p.rows_per_batch;
            g = p.gate_a[(int64_t)b * p.gate_stride + col] + (p.gate_t ? p.gate_t[col] : 0.0f);
        }
        float * xr = p.out32 + (int64_t)row * p.ldo32 + col;
        const float nx = *xr + g * v;
        *xr = nx;
        if (p.out16) reinterpret_cast<f16 *>(p.out16)[(int64_t)row * p.ldo16 + col] = (f16)nx;
    } else {
        if (p.bias) v += p.bias[col];
        if (p.act == kActSilu) v = silu_f(v);
        else if (p.act == kActGelu) v = gelu_tanh_f(v);
        if (p.out32) p.out32[(int64_t)row * p.ldo32 + col] = v;
        if (p.out16) reinterpret_cast<f16 *>(p.out16)[(int64_t)row * p.ldo16 + col] = (f16)v;
    }
}

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int AL = BM * 8 / 256, BL = BN * 8 / 256;
    __shared__ __attribute__((aligned(16))) f16 sA[2][BM * kBK];
    __shared__ __attribute__((aligned(16))) f16 sB[2][BN * kBK];

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
    const int wm = wid >> 1, wn = wid & 1;

    const f16 * aptr[AL];
    const f16 * bptr[BL];
    int alds[AL], blds[BL];
#pragma unroll
    for (int i = 0; i < AL; ++i) {
        const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
        const int gm = min(m0 + row, p.M - 1);
        aptr[i] = reinterpret_cast<const f16 *>(p.A) + (int64_t)gm * p.lda + ch * 8;
        alds[i] = swz(row, ch);
    }
#pragma unroll
    for (int i = 0; i < BL; ++i) {
        const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
        const int gn = min(n0 + row, p.N - 1);
        bptr[i] = reinterpret_cast<const f16 *>(p.W) + (int64_t)gn * p.ldw + ch * 8;
        blds[i] = swz(row, ch);
    }

    f16x8 ra[AL], rb[BL];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < AL; ++i) ra[i] = *reinterpret_cast<const f16x8 *>(aptr[i] + k0);
#pragma unroll
        for (int i = 0; i < BL; ++i) rb[i] = *reinterpret_cast<const f16x8 *>(bptr[i] + k0);
    };
    auto lstore = [&](int st) {
#pragma unroll
        for (int i = 0; i < AL; ++i) *reinterpret_cast<f16x8 *>(&sA[st][alds[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < BL; ++i) *reinterpret_cast<f16x8 *>(&sB[st][blds[i]]) = rb[i];
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int KT = p.K / kBK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * kBK);
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            const int ch = 2 * s + (lane >> 5);
            f16x8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = wm * WM + i * 32 + (lane & 31);
                af[i] = *reinterpret_cast<const f16x8 *>(&sA[cur][swz(row, ch)]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int row = wn * WN + j * 32 + (lane & 31);
                bf[j] = *reinterpret_cast<const f16x8 *>(&sB[cur][swz(row, ch)]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma_32x32x16(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < KT) lstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: lane owns column (lane & 31) of each 32x32 block and rows
    // 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < p.M && col < p.N) epilogue<MODE>(p, row, col, acc[i][j][r]);
            }
        }
    }
}

template <int BM, int BN>
hipError_t launch(const GemmParams & p, hipStream_t s) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    if (p.mode == kGemmResidual)
        hipLaunchKernelGGL((gemm_kernel<BM, BN, kGemmResidual>), dim3(tiles), dim3(256), 0, s, p);
    else if (p.mode == kGemmVT)
        hipLaunchKernelGGL((gemm_kernel<BM, BN, kGemmVT>), dim3(tiles), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_kernel<BM, BN, kGemmStore>), dim3(tiles), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm(const GemmParams & p, hipStream_t s) {
    if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % kBK != 0) return hipErrorInvalidValue;
    if (!p.A || !p.W || p.lda < p.K || p.ldw < p.K || p.lda % 8 || p.ldw % 8) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.W)) & 15) return hipErrorInvalidValue;
    if (p.mode == kGemmResidual && !p.out32) return hipErrorInvalidValue;
    if (p.mode == kGemmVT && (!p.out16 || p.vt_rows <= 0 || p.vt_cols <= 0 || p.vt_batch <= 0 ||
                              p.vt_ld < p.vt_cols || p.N != p.vt_batch * p.vt_cols || p.M % p.vt_rows))
        return hipErrorInvalidValue;
    if (p.mode == kGemmStore && !p.out16 && !p.out32) return hipErrorInvalidValue;
    if (p.gate_a && p.rows_per_batch <= 0) return hipErrorInvalidValue;
    const int64_t t256 = (int64_t)((p.M + 255) / 256) * ((p.N + 127) / 128);
    const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
    const int64_t t64 = (int64_t)((p.M + 127) / 128) * ((p.N + 63) / 64);
    if (t256 >= 320) return launch<256, 128>(p, s);
    if (t128 >= 256) return launch<128, 128>(p, s);
    if (t64 >= 200) return launch<128, 64>(p, s);
    return launch<64, 64>(p, s);
}

}  // namespace sana
