"""mxq.block._driver's layout helpers on the CPU (torch views and copies, no kernels): Blocks, to_blocks,
codes_from_blocks, scales_from_blocks against the oracle's block split and the round trip they promise."""
import numpy as np
import pytest
import torch

from _util import assert_bits_equal
from oracle import block as ob

from mxq.block import _driver


@pytest.mark.parametrize("shape, axis, bs", [((100, 40), 0, 32), ((3, 70, 5), -2, 32), ((48, 33), -1, 16),
                                             ((64, 8), 0, 32), ((5,), 0, 7), ((2, 0, 3), 1, 32)])
def test_layout_helpers(shape, axis, bs):
    rng = np.random.default_rng(len(shape) * 100 + bs)
    V = rng.standard_normal(shape).astype(np.float32)
    b = _driver.to_blocks(torch.from_numpy(V), axis, bs)
    want, want_axis, want_n = ob._to_blocks(V, axis, bs)
    assert isinstance(b, _driver.Blocks) and b.axis == want_axis and b.n == want_n
    assert_bits_equal(b.data.numpy(), want, f"to_blocks {shape}")
    assert_bits_equal(_driver.codes_from_blocks(b.data, b).numpy(), V, "codes_from_blocks round trip")
    X = b.data.abs().amax(dim=-1, keepdim=True) if b.data.shape[-1] and b.data.numel() else \
        torch.zeros(b.data.shape[:-1] + (1,))
    Xl = _driver.scales_from_blocks(X, b)
    want_shape = list(shape)
    want_shape[axis % len(shape)] = -(-shape[axis % len(shape)] // bs)
    assert list(Xl.shape) == want_shape and Xl.is_contiguous()


def test_to_blocks_keeps_dtype_and_rejects_bad_axis():
    V = torch.arange(40, dtype=torch.bfloat16).reshape(40, 1)
    b = _driver.to_blocks(V, 0, 32)
    assert b.data.dtype == torch.bfloat16 and b.data.shape == (1, 2, 32)
    assert torch.equal(b.data[0, 1, 8:], torch.zeros(24, dtype=torch.bfloat16))
    with pytest.raises(IndexError, match="axis"):
        _driver.to_blocks(V, 2, 32)


def test_lut_host_tables_against_reference_fixtures():
    """mxq.lut's host-side tables (no kernel): values, decode, and encode back to codes, against the reference's
    own outputs (tests/golden/lut_*.npz) for the four LUT formats."""
    import os

    from mxq import lut
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    for fmt in lut.FORMATS:
        z = np.load(os.path.join(golden, f"lut_{fmt}.npz"), allow_pickle=False)
        assert_bits_equal(lut.values(fmt).numpy(), z["values"], f"values {fmt}")
        dec = lut.decode(torch.from_numpy(z["decode_codes"]), fmt).numpy()
        assert_bits_equal(dec, z["decode"], f"decode {fmt}")
        finite = np.isfinite(dec)
        codes = lut.encode(torch.from_numpy(dec[finite]), fmt).numpy()
        assert_bits_equal(lut.decode(torch.from_numpy(codes), fmt).numpy(), dec[finite], f"encode {fmt}")
        first = {}
        for c, b in enumerate(dec.view(np.uint32)):
            first.setdefault(int(b), c)
        assert [first[int(b)] for b in dec[finite].view(np.uint32)] == codes.tolist(), "lowest code of each value"
        with pytest.raises(ValueError, match="not an exact"):
            lut.encode(torch.tensor([0.3]), fmt)
