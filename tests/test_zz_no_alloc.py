"""afhip_gemm_run_static, the GEMM entry point that allocates nothing, against
afhip_gemm_run with a workspace of the caller's: bit-identical outputs on two
calls in a row (the second smaller, so it reuses the array the first left
behind), a plan whose workspace exceeds the array is refused, and a plan
that needs no workspace runs too. Everything goes through the C ABI."""
import ctypes

import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    from afhip import device

    device.open_device(0)
    return torch.device("cuda", 0)


def _plan(desc):
    from afhip import _lib

    handle = ctypes.c_void_p()
    _lib.call("afhip_gemm_plan_create", ctypes.byref(desc), ctypes.byref(handle))
    size = ctypes.c_size_t()
    _lib.call("afhip_gemm_workspace_size", handle, ctypes.byref(size))
    return handle, size.value


def _desc(M, K, N, *, precision, a_dtype, w_dtype, w_layout, out_dtype, epilogue=0, batch=1, sa=0, sw=0, sc=0):
    from afhip import _lib

    return _lib.GemmDesc(M, K, N, batch, precision, a_dtype, w_dtype, w_layout, out_dtype, epilogue, 0, 0, 0, 0, 0,
                         sa, sw, sc)


def _both(dev, desc, a, w, bias, out_shape, out_dtype):
    """Runs one plan through afhip_gemm_run (fresh workspace) and through
    afhip_gemm_run_static; returns both outputs on the host."""
    import torch

    from afhip import _lib
    from afhip.device import stream_handle

    plan, ws_bytes = _plan(desc)
    try:
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        ref_out = torch.full(out_shape, float("nan"), dtype=out_dtype, device=dev)
        got = torch.full(out_shape, float("nan"), dtype=out_dtype, device=dev)
        bias_p = None if bias is None else bias.data_ptr()
        _lib.call("afhip_gemm_run", plan, a.data_ptr(), w.data_ptr(), None, bias_p, None, ref_out.data_ptr(),
                  ws.data_ptr(), ws_bytes, stream_handle())
        _lib.call("afhip_gemm_run_static", plan, a.data_ptr(), w.data_ptr(), None, bias_p, None, got.data_ptr(),
                  stream_handle())
        torch.cuda.synchronize()
        return ws_bytes, ref_out.cpu(), got.cpu()
    finally:
        _lib.library().afhip_gemm_plan_destroy(plan)


def test_static_matches_workspace_entry_point_twice(dev):
    import torch

    from afhip import _lib

    for case, (M, K, N) in enumerate([(300, 256, 520), (97, 64, 136)]):
        print(f"no-alloc f16 case {case}: M={M} K={K} N={N}", flush=True)
        a = torch.from_numpy(ref.round_f16(ref.normal(40 + case, (M, K)))).half().to(dev)
        w = torch.from_numpy(ref.round_f16(ref.normal(50 + case, (K, N), 1 / K))).half().to(dev)
        b = torch.from_numpy(ref.normal(60 + case, (N,), 0.02)).to(dev)
        desc = _desc(M, K, N, precision=_lib.PRECISION_F16, a_dtype=_lib.F16, w_dtype=_lib.F16,
                     w_layout=_lib.WEIGHT_COLUMN_CONTIGUOUS, out_dtype=_lib.F32,
                     epilogue=_lib.EPILOGUE_BIAS | _lib.EPILOGUE_RELU)
        ws_bytes, expect, got = _both(dev, desc, a, w, b, (M, N), torch.float32)
        assert ws_bytes > 0  # the column-contiguous weight goes through the scratch
        assert torch.equal(expect, got), f"case {case}"
        # and both agree with float64 at the f16 tolerance
        e64 = np.maximum(a.double().cpu().numpy() @ w.double().cpu().numpy() + b.double().cpu().numpy(), 0)
        assert np.abs(got.numpy() - e64).max() <= 1e-2 * max(1.0, np.abs(e64).max())


def test_static_f32_batched_weights(dev):
    import torch

    from afhip import _lib

    for case, (B, M, K, N) in enumerate([(3, 65, 96, 70), (2, 33, 40, 17)]):
        print(f"no-alloc f32 batched case {case}: B={B} M={M} K={K} N={N}", flush=True)
        a = torch.from_numpy(ref.normal(70 + case, (B, M, K))).to(dev)
        w = torch.from_numpy(ref.normal(80 + case, (B, K, N), 1 / K)).to(dev)
        desc = _desc(M, K, N, precision=_lib.PRECISION_F32, a_dtype=_lib.F32, w_dtype=_lib.F32,
                     w_layout=_lib.WEIGHT_COLUMN_CONTIGUOUS, out_dtype=_lib.F32, batch=B, sa=M * K, sw=K * N,
                     sc=M * N)
        ws_bytes, expect, got = _both(dev, desc, a, w, None, (B, M, N), torch.float32)
        assert ws_bytes >= B * K * N * 4
        assert torch.equal(expect, got), f"case {case}"


def test_static_without_workspace_and_refusal(dev):
    import torch

    from afhip import _lib
    from afhip.device import stream_handle

    M, K, N = 128, 64, 256
    a = torch.from_numpy(ref.round_f16(ref.normal(90, (M, K)))).half().to(dev)
    wt = torch.from_numpy(ref.round_f16(ref.normal(91, (N, K), 1 / K))).half().to(dev)
    desc = _desc(M, K, N, precision=_lib.PRECISION_F16, a_dtype=_lib.F16, w_dtype=_lib.F16,
                 w_layout=_lib.WEIGHT_K_CONTIGUOUS, out_dtype=_lib.F16)
    ws_bytes, expect, got = _both(dev, desc, a, wt, None, (M, N), torch.float16)
    assert ws_bytes == 0
    assert torch.equal(expect, got)

    limit = ctypes.c_size_t()
    _lib.call("afhip_gemm_static_scratch_bytes", ctypes.byref(limit))
    assert limit.value == 8 << 20
    # K x N f16 = 16 MiB of transposed weight: more than the array holds. The
    # entry point refuses it before launching anything.
    big = _desc(64, 4096, 2048, precision=_lib.PRECISION_F16, a_dtype=_lib.F16, w_dtype=_lib.F16,
                w_layout=_lib.WEIGHT_COLUMN_CONTIGUOUS, out_dtype=_lib.F32)
    plan, need = _plan(big)
    try:
        assert need > limit.value
        status = _lib.library().afhip_gemm_run_static(plan, a.data_ptr(), a.data_ptr(), None, None, None,
                                                      a.data_ptr(), stream_handle())
        assert status == _lib.ERR_INVALID_ARGUMENT
        assert "static scratch" in _lib.last_error()
    finally:
        _lib.library().afhip_gemm_plan_destroy(plan)
