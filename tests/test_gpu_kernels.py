"""Kernel-level parity of the gfx950 HIP kernels, called through the C ABI.

Each kernel is compared with the CPU oracle (or an fp64 numpy product for the
GEMM) evaluated on the same fp16-rounded operands, so the only differences
left are accumulation order and the fp16 rounding of the kernel's own output.
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.fixture(scope="module")
def L():
    _need_gpu()
    import sana_dit
    return sana_dit


GEMM_SHAPES = [
    (2048, 3456, 1152),   # fused QKV at 1024 px
    (2048, 5760, 1152),   # Mix-FFN inverted
    (2048, 1152, 2880),   # Mix-FFN point
    (2048, 1152, 1152),   # attention out / cross q / cross out
    (2000, 5760, 1152),   # 128x192 tiles in one round, last row tile partial
    (1000, 5760, 1152),   # 128x128 tiles, last row tile partial
    (16300, 1152, 1152),  # 128x192 tiles over many rounds, last row tile partial
    (2000, 1152, 2880),   # 128x64 tiles, last row tile partial
    (600, 4608, 1152),    # cross K of 4 blocks
    (300, 16384, 256),    # <= 5 row tiles against >= 128 column tiles: 8-wave 128x128 tiles
    (16384, 300, 256),    # the same with rows and columns swapped
    (600, 1152, 2304),    # small grid, K >= 2048: 64x64 tiles, 3 stages, early release
    (100, 70, 64),        # ragged M and N
    (7, 3, 64),           # tiny
]


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_store(L, M, N, K):
    rng = np.random.default_rng(M * 7 + N)
    A = f16(rng.standard_normal((M, K)))
    W = f16(rng.standard_normal((N, K)) * 0.03)
    bias = rng.standard_normal(N).astype(np.float32) * 0.1
    ref = A.astype(np.float64) @ W.astype(np.float64).T + bias
    dA, dW, db = dev(A, torch.float16), dev(W, torch.float16), dev(bias, torch.float32)
    o32 = torch.empty((M, N), device="cuda", dtype=torch.float32)
    o16 = torch.empty((M, N), device="cuda", dtype=torch.float16)
    L.check(L.lib().sana_hip_gemm(dA.data_ptr(), K, dW.data_ptr(), K, M, N, K, db.data_ptr(), 0, o16.data_ptr(), N,
                                  o32.data_ptr(), N, stream()))
    got32, got16 = host(o32), host(o16)
    assert rel_l2(got32, ref) < 1e-5, rel_l2(got32, ref)
    assert rel_l2(got16, ref) < 1e-3
    assert np.abs(got32 - ref).max() < 1e-3 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("act,M,N,K", [(1, 300, 200, 128), (2, 300, 200, 128),
                                       (2, 600, 1152, 2304)])   # the caption projection's GELU GEMM
def test_gemm_activation(L, act, M, N, K):
    rng = np.random.default_rng(act)
    A = f16(rng.standard_normal((M, K)))
    W = f16(rng.standard_normal((N, K)) * 0.1)
    bias = rng.standard_normal(N).astype(np.float32)
    z = A.astype(np.float64) @ W.astype(np.float64).T + bias
    ref = z / (1 + np.exp(-z)) if act == 1 else 0.5 * z * (1 + np.tanh(np.sqrt(2 / np.pi) * (z + 0.044715 * z ** 3)))
    o32 = torch.empty((M, N), device="cuda", dtype=torch.float32)
    dA, dW, db = dev(A, torch.float16), dev(W, torch.float16), dev(bias, torch.float32)
    L.check(L.lib().sana_hip_gemm(dA.data_ptr(), K, dW.data_ptr(), K, M, N, K, db.data_ptr(), act, None, 0,
                                  o32.data_ptr(), N, stream()))
    assert rel_l2(host(o32), ref) < 1e-5


@pytest.mark.parametrize("M,N,K", [(300, 200, 128), (738, 2048, 256), (5, 16, 64)])
def test_gemm_geglu_pairs(L, M, N, K):
    """act 3: W rows interleaved as gate / up pairs, the epilogue stores
    f16(gelu_tanh(gate) * up) at column n / 2 (the Gemma FFN's gating)."""
    rng = np.random.default_rng(M + N)
    A = f16(rng.standard_normal((M, K)))
    W = f16(rng.standard_normal((N, K)) * 0.1)
    z = A.astype(np.float64) @ W.astype(np.float64).T
    g, u = z[:, 0::2], z[:, 1::2]
    ref = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u
    o16 = torch.empty((M, N // 2), device="cuda", dtype=torch.float16)
    dA, dW = dev(A, torch.float16), dev(W, torch.float16)
    L.check(L.lib().sana_hip_gemm(dA.data_ptr(), K, dW.data_ptr(), K, M, N, K, None, 3, o16.data_ptr(), N // 2,
                                  None, 0, stream()))
    assert rel_l2(host(o16), ref) < 1e-3
    o32 = torch.empty((M, N), device="cuda", dtype=torch.float32)
    rc = L.lib().sana_hip_gemm(dA.data_ptr(), K, dW.data_ptr(), K, M, N, K, None, 3, o16.data_ptr(), N // 2,
                               o32.data_ptr(), N, stream())
    assert rc != 0   # gated output is fp16 only


@pytest.mark.parametrize("B,Ntok,C,K", [(2, 96, 160, 128), (2, 1000, 1152, 2880),
                                         (2, 8192, 1152, 1152)])   # 128x192 residual tiles
def test_gemm_residual_gate(L, B, Ntok, C, K):
    M = B * Ntok
    rng = np.random.default_rng(5)
    A = f16(rng.standard_normal((M, K)))
    W = f16(rng.standard_normal((C, K)) * 0.1)
    bias = rng.standard_normal(C).astype(np.float32)
    x = rng.standard_normal((M, C)).astype(np.float32)
    tmod = rng.standard_normal((B, 6 * C)).astype(np.float32)
    table = rng.standard_normal((6, C)).astype(np.float32)
    gate = tmod[:, 2 * C:3 * C] + table[2]
    y = A.astype(np.float64) @ W.astype(np.float64).T + bias
    ref = x + np.repeat(gate, Ntok, axis=0) * y
    dx = dev(x, torch.float32)
    o16 = torch.empty((M, C), device="cuda", dtype=torch.float16)
    dA, dW, db = dev(A, torch.float16), dev(W, torch.float16), dev(bias, torch.float32)
    dt, dtab = dev(tmod, torch.float32), dev(table, torch.float32)
    L.check(L.lib().sana_hip_gemm_residual(dA.data_ptr(), K, dW.data_ptr(), K, M, C, K, db.data_ptr(),
                                           dt.data_ptr() + 2 * C * 4, dtab.data_ptr() + 2 * C * 4, 6 * C, Ntok,
                                           dx.data_ptr(), C,
                                           o16.data_ptr(), C, stream()))
    got = host(dx)
    assert rel_l2(got, ref) < 1e-5
    assert rel_l2(host(o16), got) < 1e-3


def test_gemm_rejects_bad_k(L):
    M, N, K = 64, 64, 100
    a = torch.zeros((M, 128), device="cuda", dtype=torch.float16)
    o = torch.empty((M, N), device="cuda", dtype=torch.float32)
    rc = L.lib().sana_hip_gemm(a.data_ptr(), 128, a.data_ptr(), 128, M, N, K, None, 0, None, 0, o.data_ptr(), N,
                               stream())
    assert rc == L.SANA_ERR_SHAPE


@pytest.mark.parametrize("C", [1152, 2, 130])
def test_ln_modulate(L, C):
    B, N = 2, 33
    rng = np.random.default_rng(C)
    x = (rng.standard_normal((B, N, C)) * 3 + 1).astype(np.float32)
    tmod = (rng.standard_normal((B, 6 * C)) * 0.1).astype(np.float32)
    table = (rng.standard_normal((6, C)) * 0.1).astype(np.float32)
    mod = tmod + table.reshape(-1)
    ref = O.modulate(O.layer_norm(x, 1e-6), mod[:, :C], mod[:, C:2 * C])
    out = torch.empty((B * N, C), device="cuda", dtype=torch.float16)
    dx, dt, dtab = dev(x, torch.float32), dev(tmod, torch.float32), dev(table, torch.float32)
    L.check(L.lib().sana_hip_ln_modulate(dx.data_ptr(), C, out.data_ptr(), C, B * N, C, N, 1e-6, None, None,
                                         dt.data_ptr(), dtab.data_ptr(), 6 * C, 0, C, stream()))
    got = host(out).reshape(B, N, C)
    assert rel_l2(got, ref) < 1e-3


@pytest.mark.parametrize("B,N,H,D", [(2, 1024, 36, 32), (2, 4096, 16, 72), (1, 256, 16, 72), (1, 5, 1, 2),
                                     (2, 300, 3, 7), (1, 200, 4, 48), (1, 130, 2, 112), (1, 70, 3, 24),
                                     (1, 100, 2, 8), (1, 90, 2, 56), (1, 77, 2, 64), (1, 64, 2, 88)])
def test_linear_attention(L, B, N, H, D):
    rng = np.random.default_rng(N + D)
    C = H * D
    q, k, v = (f16(rng.standard_normal((B, N, C))) for _ in range(3))
    ref = O.linear_attention(q, k, v, H)
    ws = torch.empty(L.lib().sana_hip_linear_attention_workspace(B, N, H, D) // 4 + 1, device="cuda",
                     dtype=torch.float32)
    dq, dk, dv = dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16)
    out = torch.empty((B * N, C), device="cuda", dtype=torch.float16)
    L.check(L.lib().sana_hip_linear_attention(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), C, out.data_ptr(), C, B,
                                              N, H, D, ws.data_ptr(), stream()))
    got = host(out).reshape(B, N, C)
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)


@pytest.mark.parametrize("N,D,kscale,vmean,vscale", [(16384, 32, 4.0, 6.0, 1.0), (16384, 72, 4.0, 6.0, 1.0),
                                                    (64, 32, 1e-3, 0.0, 1e-3), (64, 72, 1e-3, 0.0, 1e-3)],
                         ids=["big32", "big72", "tiny32", "tiny72"])
def test_linear_attention_state_range(L, N, D, kscale, vmean, vscale):
    # |S| = |sum_t relu(k) v| ~ N * 3.2 * 6 = 3e5 (past fp16's 65504) or ~1e-5
    # (fp16 subnormal): the state's power-of-two scaling keeps both exact
    B, H = 1, 2
    rng = np.random.default_rng(N + D)
    C = H * D
    q = f16(rng.standard_normal((B, N, C)))
    k = f16(np.abs(rng.standard_normal((B, N, C))) * kscale)
    v = f16(rng.standard_normal((B, N, C)) * vscale + vmean)
    ref = O.linear_attention(q, k, v, H)
    ws = torch.empty(L.lib().sana_hip_linear_attention_workspace(B, N, H, D) // 4 + 1, device="cuda",
                     dtype=torch.float32)
    dq, dk, dv = dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16)
    out = torch.empty((B * N, C), device="cuda", dtype=torch.float16)
    L.check(L.lib().sana_hip_linear_attention(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), C, out.data_ptr(), C, B,
                                              N, H, D, ws.data_ptr(), stream()))
    got = host(out).reshape(B, N, C)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)


def test_linear_attention_negative_query_gives_zero(L):
    # relu(q) == 0 for a whole head row -> numerator 0, denominator 1e-15 -> exactly 0
    B, N, H, D = 1, 64, 2, 32
    rng = np.random.default_rng(1)
    q = f16(rng.standard_normal((B, N, H * D)))
    q[0, 5, :D] = -np.abs(q[0, 5, :D]) - 0.1
    k, v = (f16(rng.standard_normal((B, N, H * D))) for _ in range(2))
    ws = torch.empty(L.lib().sana_hip_linear_attention_workspace(B, N, H, D) // 4 + 1, device="cuda",
                     dtype=torch.float32)
    out = torch.empty((B * N, H * D), device="cuda", dtype=torch.float16)
    dq, dk, dv = dev(q, torch.float16), dev(k, torch.float16), dev(v, torch.float16)
    L.check(L.lib().sana_hip_linear_attention(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), H * D, out.data_ptr(),
                                              H * D, B, N, H, D, ws.data_ptr(), stream()))
    got = host(out)
    assert np.all(got[5, :D] == 0.0)


def _xattn(L, q, k, v, H, bias, pad=0.0):
    B, N, C = q.shape
    Lk = k.shape[1]
    D = C // H
    Lp = (Lk + 31) // 32 * 32
    vt = np.full((B, C, Lp), pad, np.float32)
    vt[:, :, :Lk] = np.transpose(v, (0, 2, 1))
    dq, dk, dvt = dev(q, torch.float16), dev(k, torch.float16), dev(vt, torch.float16)
    db = None if bias is None else dev(bias, torch.float32)
    out = torch.empty((B * N, C), device="cuda", dtype=torch.float16)
    L.check(L.lib().sana_hip_cross_attention(dq.data_ptr(), C, dk.data_ptr(), C, dvt.data_ptr(), Lp,
                                             None if db is None else db.data_ptr(), out.data_ptr(), C, B, N, Lk, H, D,
                                             stream()))
    return host(out).reshape(B, N, C)


@pytest.mark.parametrize("B,N,Lk,H,D,masked", [(2, 1024, 300, 16, 72, False), (2, 256, 300, 16, 72, True),
                                               (2, 129, 300, 16, 72, True), (1, 64, 320, 2, 96, False),
                                               (1, 100, 161, 3, 48, True), (1, 70, 33, 4, 32, False),
                                               (1, 2, 2, 1, 2, False), (1, 17, 5, 3, 12, True),
                                               (1, 130, 150, 2, 64, True), (2, 200, 100, 4, 72, False),
                                               (1, 40, 5, 2, 72, False)])
def test_cross_attention(L, B, N, Lk, H, D, masked):
    # D % 8 == 0 with <= 320 keys runs the LDS-staged kernel: D = 72 and 48
    # take the softmax denominator from the ones row of V^T, D = 32, 64 and 96
    # (multiples of 32, no padding row) sum it in registers; 5 and 33 keys
    # leave the second key half (nearly) empty.  D = 2 and 12 run the generic kernel.
    rng = np.random.default_rng(N + Lk)
    C = H * D
    q = f16(rng.standard_normal((B, N, C)))
    k = f16(rng.standard_normal((B, Lk, C)))
    v = f16(rng.standard_normal((B, Lk, C)))
    bias = None
    if masked:
        bias = np.full((B, Lk), -10000.0, np.float32)
        bias[0, :1] = 0
        if B > 1:
            bias[1, :min(Lk, 40)] = 0
    ref = O.attention(q, k, v, H, bias)
    got = _xattn(L, q, k, v, H, bias)
    assert rel_l2(got, ref) < 2e-3, rel_l2(got, ref)


@pytest.mark.parametrize("B,S,F", [(2, 32, 2880), (2, 64, 2880), (1, 37, 40), (1, 16, 64), (1, 3, 5), (2, 1, 8),
                                   (1, 6, 16), (1, 7, 24), (2, 37, 40), (1, 115, 24), (1, 128, 16),
                                   (1, 32, 4096), (1, 64, 4096), (1, 128, 2048),
                                   (1, 128, 96), (1, 113, 160), (2, 112, 96), (1, 32, 96)])
def test_dwconv_glu(L, B, S, F):
    # row segments of 4 tokens up to 1024 tokens, 8 below 12288, 16 above:
    # S = 6 and 7 (4), 37 (8) and 115 (16) leave a partial last segment, S = 1
    # and 3 a row shorter than a segment; F = 5 takes the scalar kernel; the
    # VAE's power-of-two channel counts take the 8-segment pipelined kernel
    # (1024 tokens, F = 4096) and the 8-channel row kernel (64x64 x 4096,
    # 128x128 x 2048).  From 1024 tokens per launch, F a multiple of 32 and not
    # a power of two, the LDS strip kernel, 32 columns wide and as tall (32, 16,
    # 8 or 4 rows) as still makes 720 workgroups: 64 x 64 x 2880 in a batch of
    # two takes 32-row strips, 32 x 32 x 2880 in a batch of two 8-row ones;
    # smaller grids take 4 x 32 tiles staged whole (113 x 113 and 112 x 112
    # leave partial tiles in both directions)
    _dwconv_glu_case(L, B, S, S, F)


@pytest.mark.parametrize("B,H,W,F", [(1, 64, 100, 2880), (1, 70, 64, 2880), (1, 40, 40, 2880), (1, 41, 33, 2880),
                                     (1, 70, 40, 96), (1, 96, 20, 96), (1, 40, 70, 96)])
def test_dwconv_glu_rect(L, B, H, W, F):
    # rectangular grids through the strip kernel: 32-row strips with a last
    # column strip of 4 live columns (64 x 100), 16-row strips ending in a strip
    # of 6 rows (70 x 64), 8-row strips beside a strip of 8 live columns
    # (40 x 40), and 8-row strips ending in a strip of 1 row (fewer rows than
    # the DMA runs ahead) beside a strip of 1 live column (41 x 33: whole waves
    # of the strip only load and never store); and through the 4-row tiles:
    # partial tiles (70 x 40), a grid narrower than one tile (96 x 20), 40 x 70
    _dwconv_glu_case(L, B, H, W, F)


def _dwconv_glu_case(L, B, H, W, F):
    rng = np.random.default_rng(H * 1000 + W + F)
    E = 2 * F
    x = f16(rng.standard_normal((B, H, W, E)))
    w = (rng.standard_normal((E, 3, 3)) * 0.3).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    d = O.depthwise3x3(x, w, bias)
    ref = d[..., :F] * (d[..., F:] / (1 + np.exp(-d[..., F:])))
    wt = np.ascontiguousarray(w.reshape(E, 9).T)
    dx, dw, db = dev(x, torch.float16), dev(wt, torch.float32), dev(bias, torch.float32)
    out = torch.empty((B * H * W, F), device="cuda", dtype=torch.float16)
    L.check(L.lib().sana_hip_dwconv_glu(dx.data_ptr(), E, dw.data_ptr(), db.data_ptr(), out.data_ptr(), F, B, H, W, F,
                                        stream()))
    got = host(out).reshape(B, H, W, F)
    assert rel_l2(got, ref) < 1e-3, rel_l2(got, ref)


def test_peak_kernels_do_their_work(L):
    """The roofline ceilings' kernels: the HBM copy moves every byte, the
    read-only pass sums every element, and the MFMA loop gives finite sums
    (zero with zero operands)."""
    import ctypes
    lib = L.lib()
    n = (3 << 20) + 4                       # not a multiple of the grid's thread count
    src = torch.arange(n, device="cuda", dtype=torch.float32).remainder_(7.0)
    dst = torch.zeros_like(src)
    nsink = ctypes.c_int64()
    L.check(lib.sana_hip_hbm_peak(None, None, 0, None, ctypes.byref(nsink), None))
    sink = torch.zeros(nsink.value, device="cuda", dtype=torch.float32)
    L.check(lib.sana_hip_hbm_peak(src.data_ptr(), dst.data_ptr(), n * 4, sink.data_ptr(), None, stream()))
    torch.cuda.synchronize()
    assert torch.equal(dst, src)
    L.check(lib.sana_hip_hbm_peak(src.data_ptr(), None, n * 4, sink.data_ptr(), None, stream()))
    torch.cuda.synchronize()
    assert float(sink.double().sum()) == float(src.double().sum())
    assert lib.sana_hip_hbm_peak(src.data_ptr(), None, n * 4 - 4, sink.data_ptr(), None, stream()) != 0
    wg = 8
    msink = torch.full((wg * 256,), float("nan"), device="cuda", dtype=torch.float32)
    fl = ctypes.c_double()
    for zero in (0, 1):
        L.check(lib.sana_hip_mfma_peak(wg, 3, zero, msink.data_ptr(), stream(), ctypes.byref(fl)))
        torch.cuda.synchronize()
        assert fl.value == wg * 4 * 4 * 8 * 3 * 32768
        assert torch.isfinite(msink).all()
        if zero:
            assert (msink == 0).all()
        else:
            assert (msink != 0).any()


@pytest.mark.parametrize("B,N,Lk,H,D,masked", [(2, 4096, 300, 16, 72, False), (1, 4500, 300, 16, 72, True),
                                               (1, 4099, 290, 4, 64, True), (1, 8192, 300, 2, 72, False)])
def test_cross_attention_long_sequences(L, B, N, Lk, H, D, masked):
    """From 4096 queries the staged head serves several 256-query blocks with
    an online softmax over the two key halves (ragged last blocks, masks, and
    D = 64 with the in-register denominator)."""
    rng = np.random.default_rng(N + Lk + D)
    C = H * D
    q = f16(rng.standard_normal((B, N, C)))
    k = f16(rng.standard_normal((B, Lk, C)))
    v = f16(rng.standard_normal((B, Lk, C)))
    bias = None
    if masked:
        bias = np.full((B, Lk), -10000.0, np.float32)
        bias[0, :Lk // 3] = 0
        if B > 1:
            bias[1, :7] = 0
    ref = O.attention(q, k, v, H, bias)
    got = _xattn(L, q, k, v, H, bias, pad=np.nan)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) < 2e-3, rel_l2(got, ref)


@pytest.mark.parametrize("Lk,masked", [(300, False), (300, True), (77, False)])
def test_cross_attention_ignores_vt_padding(L, Lk, masked):
    """V^T columns past the key count hold NaN: the kernel must not read them
    into the result (keys past L get zero weight and zero values)."""
    rng = np.random.default_rng(Lk + masked)
    B, N, H, D = 2, 160, 16, 72
    q = f16(rng.standard_normal((B, N, H * D)))
    k = f16(rng.standard_normal((B, Lk, H * D)))
    v = f16(rng.standard_normal((B, Lk, H * D)))
    bias = None
    if masked:
        bias = np.full((B, Lk), -10000.0, np.float32)
        bias[0, :7] = 0
        bias[1, :Lk // 2] = 0
    ref = O.attention(q, k, v, H, bias)
    got = _xattn(L, q, k, v, H, bias, pad=np.nan)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) < 2e-3, rel_l2(got, ref)
