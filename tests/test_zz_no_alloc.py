"""The allocation-free split-K entry point (m5k_gemm_i8_splitk_noalloc) against the
workspace form (m5k_gemm_i8_splitk), bit for bit, through the C ABI.

The scratch array keeps the last call's contents, so the test makes two calls in a row, the
second on a smaller problem, and checks that the first call's partials do not leak into it.
"""

from __future__ import annotations

import pytest
import torch

from m5kernels_amd import _lib

pytestmark = pytest.mark.gpu

SCRATCH_ELEMS = 16 * 1024 * 1024  # M5K_SCRATCH_ELEMS in include/m5k.h


def _operands(m, n, k, seed, device, epilogue):
    g = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).to(device)
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(device)
    sa = (torch.rand(m, generator=g) * 0.01 + 1e-3).to(device)
    sb = (torch.rand(n, generator=g) * 0.01 + 1e-3).to(device)
    extra = {"bias": None, "bias_map": None, "residual": None, "gate": None, "gate_map": None}
    if epilogue == "bias":
        extra["bias"] = torch.randn((n,), generator=g).to(device)
    elif epilogue == "gate_table":
        extra["residual"] = torch.randn((m, n), generator=g).to(torch.bfloat16).to(device)
        extra["gate"] = torch.randn((3, n), generator=g).to(torch.bfloat16).to(device)
        extra["gate_map"] = torch.tensor([i % 3 for i in range(m)], dtype=torch.int32, device=device)
    return a, b, sa, sb, extra


def _call(entry, a, b, sa, sb, extra, splits, out_dtype):
    m, k = a.shape
    n = b.shape[0]
    c = torch.full((m, n), float("nan"), dtype=out_dtype, device=a.device)
    args = [_lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(sa), _lib.ptr(sb), _lib.ptr(c), _lib.dtype_code(c),
            _lib.ptr(extra["bias"]), _lib.ptr(extra["bias_map"]), _lib.ptr(extra["residual"]), _lib.ptr(extra["gate"]),
            _lib.ptr(extra["gate_map"]), splits]
    if entry == "m5k_gemm_i8_splitk":
        ws = torch.empty((splits, m, n), dtype=torch.int32, device=a.device)
        args += [_lib.ptr(ws), ws.numel()]
    _lib.call(entry, *args, _lib.stream_of(a))
    return c


@pytest.mark.parametrize("epilogue,out_dtype", [("plain", torch.bfloat16), ("bias", torch.float32),
                                                ("gate_table", torch.bfloat16)])
def test_noalloc_matches_workspace_form_twice(epilogue, out_dtype, device):
    view = torch.int32 if out_dtype == torch.float32 else torch.int16
    # A large call, then a smaller one: the second must not see the first one's partials.
    for (m, n, k, splits), seed in (((256, 4096, 4096, 8), 1), ((128, 1536, 5376, 3), 2)):
        assert splits * m * n <= SCRATCH_ELEMS
        a, b, sa, sb, extra = _operands(m, n, k, seed, device, epilogue)
        got = _call("m5k_gemm_i8_splitk_noalloc", a, b, sa, sb, extra, splits, out_dtype)
        want = _call("m5k_gemm_i8_splitk", a, b, sa, sb, extra, splits, out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(got.view(view), want.view(view)), (m, n, k, splits)


def test_noalloc_rejects_sizes_beyond_the_scratch_array(device):
    m, n, k = 256, 8192, 256
    a, b, sa, sb, extra = _operands(m, n, k, 3, device, "plain")
    splits = SCRATCH_ELEMS // (m * n) + 1
    with pytest.raises(RuntimeError, match="scratch array"):
        _call("m5k_gemm_i8_splitk_noalloc", a, b, sa, sb, extra, splits, torch.bfloat16)


def test_noalloc_replays_under_graph_capture(device):
    """The use the header names: a warm-up call (the per-device scratch lookup happens there),
    then the call captured in a HIP graph and replayed, with eager work between replays; every
    replay must equal the workspace form bit for bit."""
    m, n, k, splits = 128, 1536, 5376, 3
    a, b, sa, sb, extra = _operands(m, n, k, 4, device, "bias")
    want = _call("m5k_gemm_i8_splitk", a, b, sa, sb, extra, splits, torch.float32)
    c = torch.empty((m, n), dtype=torch.float32, device=device)
    args = [_lib.ptr(a), _lib.ptr(b), m, n, k, _lib.ptr(sa), _lib.ptr(sb), _lib.ptr(c), _lib.dtype_code(c),
            _lib.ptr(extra["bias"]), None, None, None, None, splits]
    _lib.call("m5k_gemm_i8_splitk_noalloc", *args, _lib.stream_of(a))
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int32), want.view(torch.int32))
    graph, side = torch.cuda.CUDAGraph(), torch.cuda.Stream(device=device)
    with torch.cuda.graph(graph, stream=side):
        _lib.call("m5k_gemm_i8_splitk_noalloc", *args, _lib.stream_of(a))
    other = _operands(256, 2048, 1024, 5, device, "plain")
    for _ in range(3):
        c.fill_(float("nan"))
        _call("m5k_gemm_i8_splitk_noalloc", *other, 4, torch.bfloat16)  # eager use of the scratch between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c.view(torch.int32), want.view(torch.int32))
