"""sana_hip_linear_attention_noalloc (static per-GPU scratch, no allocation)
against sana_hip_linear_attention with a caller workspace: the same kernels,
so the outputs must be bit-identical.  Two calls in a row, the second smaller
(the scratch keeps the first call's contents), and the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _run_both(L, B, N, H, D, seed):
    lib = L.lib()
    g = torch.Generator(device="cuda").manual_seed(seed)
    C = H * D
    ld = C + 8 if C % 8 == 0 else C      # a row stride wider than the heads
    q, k, v = (torch.randn((B * N, ld), device="cuda", dtype=torch.float16, generator=g) for _ in range(3))
    ref = torch.full((B * N, C), float("nan"), device="cuda", dtype=torch.float16)
    got = torch.full((B * N, C), float("nan"), device="cuda", dtype=torch.float16)
    ws = torch.empty(lib.sana_hip_linear_attention_workspace(B, N, H, D) // 4 + 1, device="cuda",
                     dtype=torch.float32)
    s = torch.cuda.current_stream().cuda_stream
    print(f"linear attention B={B} N={N} H={H} D={D}: workspace entry point", flush=True)
    L.check(lib.sana_hip_linear_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), ld, ref.data_ptr(), C, B, N, H,
                                          D, ws.data_ptr(), s))
    print(f"linear attention B={B} N={N} H={H} D={D}: no-alloc entry point", flush=True)
    L.check(lib.sana_hip_linear_attention_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), ld, got.data_ptr(), C, B,
                                                  N, H, D, s))
    torch.cuda.synchronize()
    assert torch.isfinite(ref.float()).all()
    assert torch.equal(got, ref)


def test_linear_attention_noalloc_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible to torch")
    import sana_dit as L
    _run_both(L, 2, 4096, 16, 72, 11)     # the 16x72-head microbenchmark shape
    _run_both(L, 1, 1000, 4, 40, 12)      # smaller, ragged: the scratch holds the first call's data


def test_linear_attention_noalloc_rejects_oversize():
    import sana_dit as L
    lib = L.lib()
    B, N, H, D = 4, 4096, 32, 72
    assert lib.sana_hip_linear_attention_workspace(B, N, H, D) > 16 << 20
    rc = lib.sana_hip_linear_attention_noalloc(None, None, None, H * D, None, H * D, B, N, H, D, None)
    assert rc == L.SANA_ERR_INVALID_ARGUMENT
    assert b"scratch" in lib.sana_dit_last_error()
