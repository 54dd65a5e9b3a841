"""Split-K exchange when a split ran on another XCD.

On MI355X the placement the XCD-local exchange relies on always holds, so the
recompute path (the last arrival recomputes a split whose partial sits in
another XCD's L2) is driven here by the test switch MCQ4_SPLIT_FOREIGN, which
makes the kernels treat the masked splits as foreign.  Each kernel that uses the
exchange must then still give the oracle's result (the recompute sums in fp32
too, so results stay within the usual bar of the default path's), and the
library's fallback counter must count the recomputed tiles.
"""
import numpy as np
import pytest
import torch

from oracle import int4_ref as R4
from oracle import q4_0_ref as R

pytestmark = pytest.mark.gpu


def _rows_close(Y, Yref, tol=1e-2):
    Y = np.asarray(Y, np.float64)
    Yref = np.asarray(Yref, np.float64)
    assert np.isfinite(Y).all()
    err = np.abs(Y - Yref).max(axis=1)
    assert (err <= tol * np.abs(Yref).max(axis=1)).all(), f"max err {err.max()}"


def _q4_case(dev, M, K, N):
    import metalops_amd as mo
    g = torch.Generator().manual_seed(M + K + N)
    W = torch.randn(K, N, generator=g) * 0.02
    X = torch.randn(M, K, generator=g).half()
    blocks = R.quantize_llama_rule(W.numpy())
    b = torch.from_numpy(blocks).to(dev)
    return (lambda: mo.matmul_ggml_q4_0(X.to(dev), b)), R.matmul_f32(X.numpy(), blocks)


def _i4_case(dev, M, K, N, gs, wb):
    import metalops_amd as mo
    g = torch.Generator().manual_seed(M + K + N)
    X = torch.randn(M, K, generator=g).half().to(dev)
    if wb == 4:
        W = (torch.randn(K, N, generator=g) * 0.02).half().to(dev)    # fp16 scales/zeros
        p, s, z = mo.quantize_int4(W, gs)
        Yref = R4.matmul_f32(X.float().cpu().numpy(), p.cpu().numpy(), s.float().cpu().numpy(),
                             z.float().cpu().numpy(), gs)
        return (lambda: mo.matmul_int4(X, p, s, z, gs)), Yref
    q = torch.randint(-128, 128, (K, N), generator=g, dtype=torch.int8)
    s = (torch.rand(K // gs, N, generator=g) * 0.02).half()
    z = torch.randint(-4, 4, (K // gs, N), generator=g).half()
    Yref = R4.matmul_int8_f32(X.float().cpu().numpy(), q.numpy(), s.float().numpy(), z.float().numpy(), gs)
    args = [t.to(dev) for t in (q, s, z)]
    return (lambda: mo.matmul_int8(X, *args, gs)), Yref


def _rms_case(dev, M, K, N, gs):
    """fused_rmsnorm_linear_int4: the one-launch M == 1 kernel normalises the row
    inside the GEMV, so its recompute path must rebuild the normalised row."""
    import metalops_amd as mo
    g = torch.Generator().manual_seed(M + K + N + 1)
    X = torch.randn(M, K, generator=g).half()
    wn = (torch.rand(K, generator=g) + 0.5).half()
    W = (torch.randn(K, N, generator=g) * 0.02).half().to(dev)
    p, s, z = mo.quantize_int4(W, gs)
    Xn = R4.rmsnorm_f16(X.numpy(), wn.numpy(), 1e-5)
    Yref = R4.matmul_f32(Xn.astype(np.float32), p.cpu().numpy(), s.float().cpu().numpy(),
                         z.float().cpu().numpy(), gs)
    Xd, wnd = X.to(dev), wn.to(dev)
    return (lambda: mo.fused_rmsnorm_linear_int4(Xd, wnd, p, s, z, 1e-5, gs)), Yref


CASES = [
    # (name, environment, case builder args)
    ("q4_gemvm_s2", {"MCQ4_GEMVM_SPLIT": "2"}, ("q4", 16, 14336, 4096)),
    ("q4_gemvm_s8", {"MCQ4_GEMVM_SPLIT": "8"}, ("q4", 12, 2048, 1032)),
    ("q4_gemvm_rows4_s4", {"MCQ4_GEMVM_SPLIT": "4"}, ("q4", 3, 4096, 1040)),
    ("q4_gemvm_rows8_s2", {"MCQ4_GEMVM_SPLIT": "2"}, ("q4", 7, 11008, 512)),
    ("q4_gemm6_s2", {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "2"}, ("q4", 300, 4096, 640)),
    ("q4_gemm8_s2", {"MCQ4_GEMM_PATH": "8"}, ("q4", 300, 4096, 640)),
    # 64-column spans over K splits (q4_gemv_span.hip): 4, 5 and 4 splits, 16, 4 and 8 rows.
    ("q4_span_split_s4", {}, ("q4", 16, 14336, 4096)),
    ("q4_span_split_rows4_s5", {"MCQ4_GEMV_SPAN": "1"}, ("q4", 3, 2080, 2048)),
    ("q4_span_split_rows8", {}, ("q4", 6, 11008, 4096)),
    ("i4_gemv1", {}, ("i4", 1, 4096, 4096, 128, 4)),
    ("i4_gemv1_mr", {}, ("i4", 8, 11008, 4096, 128, 4)),
    ("i4_gemv1_rmsnorm", {}, ("rms", 1, 4096, 4096, 128)),
    ("i4_gemv", {"MCQ4_I4_GEMV1": "0"}, ("i4", 4, 4096, 1040, 64, 4)),
    ("i8_gemv", {"MCQ4_I4_GEMV1": "0"}, ("i4", 8, 4096, 1024, 128, 8)),
    ("i4_gemm6_s2", {"MCQ4_I4_GEMM7": "0"}, ("i4", 2048, 14336, 4096, 128, 4)),
]


@pytest.mark.parametrize("name,env,case", CASES, ids=[c[0] for c in CASES])
def test_split_recompute_path(dev, monkeypatch, name, env, case):
    from metalops_amd import _lib
    print(f"split recompute {name} {case}", flush=True)
    for k in ("MCQ4_GEMVM_SPLIT", "MCQ4_GEMM_PATH", "MCQ4_GEMM6_SPLIT", "MCQ4_GEMM8_SPLIT", "MCQ4_I4_GEMV1", "MCQ4_XCD_LOCAL",
              "MCQ4_SPLIT_FOREIGN", "MCQ4_I4_PATH", "MCQ4_I4_SPW1", "MCQ4_I4_GEMM7", "MCQ4_GEMV_SPAN",
              "MCQ4_SPLIT_SPIN"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    build = {"q4": _q4_case, "i4": _i4_case, "rms": _rms_case}[case[0]]
    fn, Yref = build(dev, *case[1:])
    Y = fn()
    torch.cuda.synchronize()
    base = _lib.split_fallback_count(reset=True)
    assert base == 0, "the default placement should never need the recompute path"
    monkeypatch.setenv("MCQ4_SPLIT_FOREIGN", "0xffff")
    Yf = fn()
    torch.cuda.synchronize()
    assert _lib.split_fallback_count(reset=True) > 0, "the recompute path did not run"
    monkeypatch.delenv("MCQ4_SPLIT_FOREIGN")
    _rows_close(Y.float().cpu().numpy(), Yref)
    _rows_close(Yf.float().cpu().numpy(), Yref)
    # and the next default call is unaffected (counters left zero)
    Y2 = fn()
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))


# Kernels whose XCD-local exchange waits on per-split flags (a bounded number of
# polls, then the split is recomputed).
FLAG_CASES = [
    ("i4_gemv1", ("i4", 1, 4096, 4096, 128, 4)),
    ("i4_gemv1_mr", ("i4", 8, 11008, 4096, 128, 4)),
    ("i4_gemv1_rmsnorm", ("rms", 1, 4096, 4096, 128)),
    ("i8_gemv1", ("i4", 4, 4096, 4096, 128, 8)),
    ("q4_span_split_s4", ("q4", 16, 14336, 4096)),
    ("q4_span_split_rows8", ("q4", 6, 11008, 4096)),
    ("q4_gemvm_rb2_s2", ("q4", 32, 14336, 4096)),
    ("q4_gemvm_s8", ("q4", 12, 2048, 1032), {"MCQ4_GEMVM_SPLIT": "8"}),
]


@pytest.mark.parametrize("name,case,env", [(c[0], c[1], c[2] if len(c) > 2 else {}) for c in FLAG_CASES],
                         ids=[c[0] for c in FLAG_CASES])
def test_split_flag_timeout_recomputes(dev, monkeypatch, name, case, env):
    """MCQ4_SPLIT_SPIN=0: the summing workgroup stops waiting at once and
    recomputes every other split from the inputs.  The result keeps the oracle's
    bar, the fallback counter counts the tiles, and the flags stay usable: the
    next default call gives the first call's bits with no fallback."""
    from metalops_amd import _lib
    print(f"split flag timeout {name} {case}", flush=True)
    for k in ("MCQ4_I4_GEMV1", "MCQ4_XCD_LOCAL", "MCQ4_SPLIT_FOREIGN", "MCQ4_SPLIT_SPIN", "MCQ4_I4_PATH",
              "MCQ4_I4_SPW1", "MCQ4_GEMV_SPAN", "MCQ4_GEMVM_SPLIT"):
        monkeypatch.delenv(k, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    build = {"q4": _q4_case, "i4": _i4_case, "rms": _rms_case}[case[0]]
    fn, Yref = build(dev, *case[1:])
    Y = fn()
    torch.cuda.synchronize()
    assert _lib.split_fallback_count(reset=True) == 0
    monkeypatch.setenv("MCQ4_SPLIT_SPIN", "0")
    Yt = fn()
    torch.cuda.synchronize()
    assert _lib.split_fallback_count(reset=True) > 0, "the recompute path did not run"
    monkeypatch.delenv("MCQ4_SPLIT_SPIN")
    _rows_close(Yt.float().cpu().numpy(), Yref)
    Y2 = fn()
    torch.cuda.synchronize()
    assert _lib.split_fallback_count(reset=True) == 0
    assert torch.equal(Y.view(torch.int16), Y2.view(torch.int16))


# (kernel with flags, a split-K kernel whose partials cover those flag words)
SURVIVE = [
    # INT4 decode: 32 tiles x 8 splits, flags 128 KiB into the partial area; the
    # span split form stores 1 MiB of partials there.
    ("i4_gemv1", ("i4", 1, 4096, 4096, 128, 4), {}, ("q4", 16, 14336, 4096)),
    # Span split form: flags 1 MiB in; gemm6 with two splits stores 2.3 MiB (9 tiles x 2 x 128 KiB).
    ("q4_span_split", ("q4", 16, 14336, 4096), {"MCQ4_GEMM_PATH": "6", "MCQ4_GEMM6_SPLIT": "2"},
     ("q4", 300, 4096, 640)),
]


@pytest.mark.parametrize("name,case,other_env,other", SURVIVE, ids=[c[0] for c in SURVIVE])
def test_split_flags_survive_other_kernels(dev, monkeypatch, name, case, other_env, other):
    """The flags sit behind a kernel's partials in the shared workspace, where
    other split-K kernels store their own partials between its launches.  Each
    launch reads the flags' values when it starts, so whatever was left there,
    every launch must give the same bits without a fallback."""
    from metalops_amd import _lib
    print(f"split flags survive {name} {case} {other}", flush=True)
    for k in ("MCQ4_I4_GEMV1", "MCQ4_XCD_LOCAL", "MCQ4_SPLIT_FOREIGN", "MCQ4_SPLIT_SPIN", "MCQ4_I4_PATH",
              "MCQ4_I4_SPW1", "MCQ4_GEMV_SPAN", "MCQ4_GEMVM_SPLIT", "MCQ4_GEMM_PATH", "MCQ4_GEMM6_SPLIT"):
        monkeypatch.delenv(k, raising=False)
    for k, v in other_env.items():
        monkeypatch.setenv(k, v)
    build = {"q4": _q4_case, "i4": _i4_case}
    fn, _ = build[case[0]](dev, *case[1:])
    fo, _ = build[other[0]](dev, *other[1:])
    first = fn()
    torch.cuda.synchronize()
    _lib.split_fallback_count(reset=True)
    for _ in range(5):
        fo()
        Y = fn()
        torch.cuda.synchronize()
        assert torch.equal(first.view(torch.int16), Y.view(torch.int16))
    assert _lib.split_fallback_count(reset=True) == 0


@pytest.mark.parametrize("kind,M,K,N", [("i4", 1, 4096, 4096), ("i4", 8, 11008, 4096), ("q4", 16, 14336, 4096),
                                        ("q4", 4, 11008, 4096), ("q4", 32, 14336, 4096)])
def test_split_flags_any_start_value(dev, kind, M, K, N):
    """Split flags need no initial value: a caller's workspace whose counter area
    is zero and whose every other byte is 0xFF (each flag word 0xFFFFFFFF, so the
    first step of 8 wraps past 2^32) gives the library's own workspace's bits on
    every call, with no split recomputed."""
    import metalops_amd as mo
    from metalops_amd import _lib
    print(f"split flags start value {kind} {M}x{K}x{N}", flush=True)
    lib = _lib.lib
    g = torch.Generator().manual_seed(M + K + N + 7)
    X = torch.randn(M, K, generator=g).half().to(dev)
    stream = torch.cuda.current_stream().cuda_stream
    if kind == "i4":
        W = (torch.randn(K, N, generator=g) * 0.02).half().to(dev)
        p, s, z = mo.quantize_int4(W, 128)
        want = mo.matmul_int4(X, p, s, z, 128)
        need = int(lib.mcq4_matmul_int4_workspace_bytes(M, K, N, 128, _lib.MCQ4_DTYPE_F16))

        def call(Y, ws):
            return lib.mcq4_matmul_int4(X.data_ptr(), _lib.MCQ4_DTYPE_F16, K, p.data_ptr(), s.data_ptr(),
                                        z.data_ptr(), _lib.MCQ4_DTYPE_F16, Y.data_ptr(), N, M, K, N, 128,
                                        ws.data_ptr(), ws.numel(), stream)
    else:
        W = torch.randn(K, N, generator=g) * 0.02
        b = torch.from_numpy(R.quantize_llama_rule(W.numpy())).to(dev)
        want = mo.matmul_ggml_q4_0(X, b)
        need = int(lib.mcq4_matmul_workspace_bytes(M, K, N))

        def call(Y, ws):
            return lib.mcq4_matmul_q4_0_f16(X.data_ptr(), K, b.data_ptr(), Y.data_ptr(), N, M, K, N,
                                            ws.data_ptr(), ws.numel(), stream)
    counters = 256 * 1024
    assert need > counters, "this shape splits K"
    ws = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    ws[:counters].zero_()
    torch.cuda.synchronize()
    _lib.split_fallback_count(reset=True)
    for _ in range(3):
        Y = torch.empty(M, N, dtype=torch.float16, device=dev)
        assert call(Y, ws) == _lib.MCQ4_OK
        torch.cuda.synchronize()
        assert torch.equal(want.view(torch.int16), Y.view(torch.int16))
    assert _lib.split_fallback_count(reset=True) == 0
