"""The device quantizers (qwm_quantize) produce the same bytes as ggml's CPU
model-file quantizers (restated by the oracle, which is pinned to the
reference build): Q4_K with its make_qkx2_quants search, and Q8_0."""
import numpy as np
import pytest

from tests.helpers import I64, Q80_BYTES, oracle, ptr, quantize_q4_K

torch = pytest.importorskip("torch")
import questwend_amd as qa  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    qa.lib()


@pytest.mark.parametrize("scale", [0.02, 1.0, 30.0])
def test_q4_K_device_quantizer_bytes(dev, scale):
    rng = np.random.default_rng(int(scale * 100) + 1)
    x = (rng.standard_normal((4096, 256)) * scale).astype(np.float32)
    x[::7] = np.abs(x[::7])
    x[3::11] = 0
    x[5::13, :100] = 0
    exp = quantize_q4_K(x)
    dx = torch.from_numpy(x).cuda()
    out = torch.zeros(exp.size, dtype=torch.uint8, device="cuda")
    qa.check(qa.lib().qwm_quantize(qa.TYPE_Q4_K, dx.data_ptr(), out.data_ptr(), x.size, None))
    got = out.cpu().numpy()
    bad = (got.reshape(-1, 144) != exp.reshape(-1, 144)).any(1)
    assert bad.sum() == 0, f"{bad.sum()} of {bad.size} blocks differ"


def test_q8_0_device_quantizer_bytes(dev):
    rng = np.random.default_rng(9)
    x = rng.standard_normal(1 << 20).astype(np.float32)
    x[:32] = 0
    x[32:64] = np.arange(32) - 15.5
    exp = np.zeros(x.size // 32 * Q80_BYTES, np.uint8)
    oracle().qwo_quantize_q8_0_ref(ptr(x), ptr(exp), I64(x.size))
    dx = torch.from_numpy(x).cuda()
    out = torch.zeros(exp.size, dtype=torch.uint8, device="cuda")
    qa.check(qa.lib().qwm_quantize(qa.TYPE_Q8_0, dx.data_ptr(), out.data_ptr(), x.size, None))
    assert np.array_equal(out.cpu().numpy(), exp)
