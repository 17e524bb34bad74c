"""Operands of 2 GiB and more, and the rotate() default, through the C ABI.

Each GEMM workgroup addresses only its own 256 rows of A and B through 32-bit buffer windows,
so operand size is not limited by the 32-bit buffer offset: the main loop is the same one that
every other test exercises.  Sampled rows at the far end of each operand (byte offsets past
2^31) are bit-exact against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bits_of, np_of
from m5kernels_amd import gemm, rotate
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def _far_rows(m):
    return np.array([0, 1, m // 2, m - 257, m - 256, m - 2, m - 1])


def test_int8_a_operand_over_2gib(device):
    m, k, n = 139_264, 16_384, 256  # A is 2.125 GiB
    assert m * k >= 2**31
    g = torch.Generator(device=device).manual_seed(1)
    a = torch.randint(-127, 128, (m, k), generator=g, device=device, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=g, device=device, dtype=torch.int8)
    sa = torch.rand(m, generator=g, device=device) * 0.01 + 1e-3
    sb = torch.rand(n, generator=g, device=device) * 0.01 + 1e-3
    y = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    rows = _far_rows(m)
    expected = ref.c_i8_epilogue(ref.c_gemm_i8_acc(np_of(a[rows]), np_of(b)), np_of(sa[rows]), np_of(sb))
    np.testing.assert_array_equal(bits_of(y[rows]), expected)
    del a


def test_int8_weight_over_2gib_split_k_routing(device):
    """Short M with a 2 GiB weight: gemm() plans split-K (n * k >= 2^31), which the library
    accepts now that each workgroup addresses a 256-row window."""
    from m5kernels_amd.hip import splitk_plan

    m, n, k = 16, 16_384, 131_072  # W is 2 GiB
    assert n * k >= 2**31 and splitk_plan(m, n, k) > 1
    g = torch.Generator(device=device).manual_seed(2)
    a = torch.randint(-127, 128, (m, k), generator=g, device=device, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=g, device=device, dtype=torch.int8)
    sa = torch.rand(m, generator=g, device=device) + 0.5
    sb = torch.rand(n, generator=g, device=device) + 0.5
    y = gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
    cols = _far_rows(n)
    expected = ref.c_i8_epilogue(ref.c_gemm_i8_acc(np_of(a), np_of(b[cols])), np_of(sa), np_of(sb[cols]))
    np.testing.assert_array_equal(bits_of(y[:, cols]), expected)
    del b


def test_bf16_operand_over_2gib(device):
    m, k, n = 66_000, 16_384, 128  # A is 2.01 GiB of BF16
    assert m * k * 2 >= 2**31
    g = torch.Generator(device=device).manual_seed(3)
    a = torch.randn((m, k), generator=g, device=device).to(torch.bfloat16)
    b = torch.randn((n, k), generator=g, device=device).to(torch.bfloat16)
    y = gemm(a, b, "bf16")
    rows = _far_rows(m)
    exact = a[rows].double().cpu().numpy() @ b.double().cpu().numpy().T
    assert ref.metrics(np_of(y[rows]), exact)["relative_l2"] < 1e-5
    del a


def test_rotate_default_implementation_is_the_kernel(device):
    """rotate()'s default implementation is "metal" as in the reference (hadamard.py:33); on
    MI355X that names the gfx950 kernel, as does the alias "hip"."""
    rng = np.random.default_rng(4)
    x = torch.from_numpy(rng.standard_normal((5, 512), dtype=np.float32)).to(device).to(torch.bfloat16)
    signs = torch.from_numpy(ref.hadamard_signs(512, 3)).to(device)
    y = rotate(x, 128, signs)
    assert torch.equal(y, rotate(x, 128, signs, implementation="metal"))
    assert torch.equal(y, rotate(x, 128, signs, implementation="hip"))
    np.testing.assert_array_equal(np_of(y), ref.c_hadamard_f32(x.float().cpu().numpy(), 128, np_of(signs)))
