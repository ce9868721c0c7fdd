"""GPU parity of the block formats: dequantization (GGUF layout and the repacked backend layout)
bit-exact against the oracle, and the device encoders byte-exact against the oracle's."""
import numpy as np
import pytest

import oracle as O
from tests.helpers import ALL_TYPES, TYPES, random_blocks

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("name", list(ALL_TYPES))
def test_dequant_gguf_bit_exact(gpu, name):
    from smallmind_amd.quantization import dequantize
    qt = ALL_TYPES[name]
    be = O.BLOCK_ELEMS[qt]
    for seed, nblocks in [(1, 1), (2, 7), (3, 333)]:
        b = random_blocks(qt, nblocks, seed)
        n = nblocks * be
        ref = O.dequant(qt, b, n)
        got = dequantize(qt, _dev(b), n).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (name, seed)
    if be == 1:
        return
    # a ragged tail (last block partially used), as the reference loops handle it
    b = random_blocks(qt, 3, 9)
    n = 3 * be - 5
    assert np.array_equal(dequantize(qt, _dev(b), n).cpu().numpy().view(np.uint32),
                          O.dequant(qt, b, n).view(np.uint32))


def test_dequant_f16_all_patterns(gpu):
    from smallmind_amd.quantization import dequantize
    h = np.arange(65536, dtype=np.uint16)
    got = dequantize(O.F16, _dev(h.view(np.uint8)), 65536).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, O.dequant(O.F16, h.view(np.uint8), 65536).view(np.uint32))


@pytest.mark.parametrize("name", list(ALL_TYPES))
@pytest.mark.parametrize("rows,cols", [(3, 256), (64, 2048), (17, 5632)])
def test_weight_to_float32_bit_exact_after_repack(gpu, name, rows, cols):
    """IWeightTensor.ToFloat32 of the repacked backend layout equals the reference decode of
    the original upload bytes, for random bytes in every field."""
    from smallmind_amd.quantization import GpuWeightTensor
    qt = ALL_TYPES[name]
    nb = rows * cols // O.BLOCK_ELEMS[qt]
    b = random_blocks(qt, nb, rows * 31 + cols)
    w = GpuWeightTensor(qt, rows, cols, b)
    got = w.to_float32().cpu().numpy().reshape(-1)
    ref = O.dequant(qt, b, rows * cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w.close()


@pytest.mark.parametrize("name", list(TYPES) + ["SMQ_Q8", "SMQ_Q4", "F16"])
def test_device_encoder_matches_oracle_bytes(gpu, name):
    from smallmind_amd.quantization import quantize
    qt = ALL_TYPES[name]
    rng = np.random.default_rng(qt)
    x = np.concatenate([rng.normal(0, 0.02, 256 * 40), rng.normal(0, 3, 256 * 8),
                        np.zeros(256), np.full(256, 1e-6), rng.uniform(-1, 1, 256)]).astype(np.float32)
    # exact ties for the rounding path
    x[:64] = (np.arange(64) - 32) * 0.5
    got = quantize(qt, _dev(x)).cpu().numpy()
    assert np.array_equal(got, O.quantize(qt, x))


def test_fill_normal_statistics(gpu):
    from smallmind_amd.quantization import fill_normal
    v = fill_normal(5, 1_000_001, 0.02).cpu().numpy().astype(np.float64)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 1e-4
    w = O.fill_normal(5, 1001, 0.02)
    assert np.allclose(fill_normal(5, 1001, 0.02).cpu().numpy(), w, rtol=1e-5, atol=1e-8)


def test_quantize_roundtrip_on_device(gpu):
    from smallmind_amd.quantization import dequantize, quantize
    rng = np.random.default_rng(0)
    v = rng.normal(0, 0.02, 4096).astype(np.float32)
    b = quantize(O.Q8_0, _dev(v))
    y = dequantize(O.Q8_0, b, 4096).cpu().numpy()
    assert np.abs(y - v).max() < np.abs(v).max() / 127
