"""GPU parity of the block-Hadamard rotation and the fused rotation + INT8 quantizer.

Bars: FP32 rotation bit-exact against the oracle's fixed-order FP32 butterflies, and
within rtol 2e-5 of the float64 definition (the reference's own gate,
tests/test_hadamard_metal.py:18-33 of the reference); fused codes/scales bit-exact against
quantize(rotate(x)).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import np_of
from m5kernels_amd import quantize, rotate, rotate_quantize
from oracle import reference as ref

pytestmark = pytest.mark.gpu

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.mark.parametrize("block", [32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_rotate_bit_exact_and_reference_gate(block, dtype, device):
    rng = np.random.default_rng(19)
    x = rng.standard_normal((5, 3 * block), dtype=np.float32)
    x[:, ::block] *= 100
    xt = torch.from_numpy(x).to(device).to(DTYPES[dtype])
    signs = ref.hadamard_signs(3 * block, 17)
    y = rotate(xt, block, torch.from_numpy(signs).to(device))
    assert y.dtype == torch.float32
    x32 = xt.float().cpu().numpy()
    np.testing.assert_array_equal(np_of(y), ref.c_hadamard_f32(x32, block, signs))
    np.testing.assert_allclose(np_of(y), ref.block_hadamard_reference(x32, block, signs), rtol=2e-5, atol=1e-5)


@pytest.mark.parametrize("block", [32, 128, 256, 512, 1024])
@pytest.mark.parametrize("dtype", list(DTYPES))
def test_rotate_ragged_grid(block, dtype, device):
    """37 rows of 2 blocks: the last workgroup's second tile slab ends mid-grid (lanes past the
    end rotate zeros and store nothing), for 4-element tiles and for grouped tiles (B >= 512)."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal((37, 2 * block), dtype=np.float32)
    xt = torch.from_numpy(x).to(device).to(DTYPES[dtype])
    signs = ref.hadamard_signs(2 * block, 5)
    y = rotate(xt, block, torch.from_numpy(signs).to(device))
    np.testing.assert_array_equal(np_of(y), ref.c_hadamard_f32(xt.float().cpu().numpy(), block, signs))


@pytest.mark.parametrize("block", [128, 256])
def test_rotate_ffn_down_shape(block, device):
    g = torch.Generator(device="cpu").manual_seed(29)
    a = torch.randn((4096, 16384), generator=g)
    a[:, ::1024] *= 50
    at = a.to(device).to(torch.bfloat16)
    signs = ref.hadamard_signs(16384, 7)
    y = rotate(at, block, torch.from_numpy(signs).to(device))
    rows = ref.sample_indices(4096)
    np.testing.assert_array_equal(np_of(y)[rows], ref.c_hadamard_f32(at.float().cpu().numpy()[rows], block, signs))
    # size-independent property: the orthonormal transform preserves every row norm
    ratio = (y.double().norm(dim=1) / at.double().norm(dim=1)).cpu().numpy()
    np.testing.assert_allclose(ratio, 1.0, rtol=1e-5)


@pytest.mark.parametrize("block", [32, 128, 256, 1024])
@pytest.mark.parametrize(
    "shape",
    [(7, 5376 // 256 * 256), (3, 4096), (3, 6144), (2, 8192), (2, 16384), (5, 1024), (2, 20480), (1, 32768)],
)
def test_fused_rotate_quantize_equals_composition(block, shape, device):
    """Every register layout of the fused kernel: 256 threads with 1-4 chunks, 512 x 2 or 4 and
    1024 x 2 or 4 chunks per thread, full and ragged rows (K 20480 leaves chunks idle)."""
    if shape[1] % block:
        pytest.skip("K not divisible by block")
    rng = np.random.default_rng(31)
    x = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(device).to(torch.bfloat16)
    signs = torch.from_numpy(ref.hadamard_signs(shape[1], 13)).to(device)
    q, s = rotate_quantize(x, block, signs)
    rq, rs = quantize(rotate(x, block, signs), "int8")
    assert torch.equal(q, rq) and torch.equal(s, rs)
    oq, os_ = ref.quantize_reference(ref.c_hadamard_f32(x.float().cpu().numpy(), block, np_of(signs)), "int8")
    np.testing.assert_array_equal(np_of(q), oq)
    np.testing.assert_array_equal(np_of(s), os_)


def test_fused_rotate_quantize_row_limit(device):
    """Rows past the register-resident limit (4096 chunks of 8 at H128) are refused with the
    library's message, before any launch."""
    x = torch.zeros((1, 65536), dtype=torch.bfloat16, device=device)
    signs = torch.ones(65536, dtype=torch.int8, device=device)
    with pytest.raises(RuntimeError, match="register-resident row limit"):
        rotate_quantize(x, 128, signs)


def test_zero_rows_and_dot_preservation(device):
    a = torch.zeros((3, 512), device=device, dtype=torch.bfloat16)
    signs = torch.from_numpy(ref.hadamard_signs(512, 3)).to(device)
    q, s = rotate_quantize(a, 128, signs)
    assert torch.all(q == 0) and torch.all(s == 1)
    rng = np.random.default_rng(21)
    x = torch.from_numpy(rng.standard_normal((4, 512), dtype=np.float32)).to(device)
    w = torch.from_numpy(rng.standard_normal((6, 512), dtype=np.float32)).to(device)
    rx, rw = rotate(x, 128, signs), rotate(w, 128, signs)
    np.testing.assert_allclose((rx.double() @ rw.double().T).cpu().numpy(), (x.double() @ w.double().T).cpu().numpy(),
                               rtol=1e-5, atol=1e-4)


def test_strided_input_not_mutated(device):
    base = torch.randn(8, 1024, device=device)
    view = base[:, ::2]
    before = base.clone()
    signs = torch.ones(512, dtype=torch.int8, device=device)
    y = rotate(view, 256, signs)
    np.testing.assert_array_equal(np_of(y), ref.c_hadamard_f32(view.cpu().numpy(), 256, np.ones(512, np.int8)))
    assert torch.equal(base, before)


@pytest.mark.parametrize("block", [64, 128, 256])
def test_rotate_quantize_extreme_rows_bit_exact(block, device):
    """The folded 1/sqrt(B) encoder on rows far from unit scale: peaks that put the reciprocal
    scale outside the fast range (the whole row takes the exact chain), a zero row, and an
    ordinary row.  Codes and scales equal quantize(c_hadamard_f32(x)) bit for bit."""
    rng = np.random.default_rng(block)
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    x[0] *= np.float32(1e-33)
    x[1] *= np.float32(1e35)
    x[2] = 0.0
    x[3] *= np.float32(1e-30)
    xt = torch.from_numpy(x).to(device)
    signs = torch.from_numpy(ref.hadamard_signs(2048, 3)).to(device)
    q, s = rotate_quantize(xt, block, signs)
    rq, rs = ref.quantize_reference(ref.c_hadamard_f32(x, block, np_of(signs)), "int8")
    np.testing.assert_array_equal(np_of(q), rq)
    np.testing.assert_array_equal(np_of(s), rs)
