"""GPU: the canary KL kernel against the reference's own outputs and the float64
oracle; batched layers equal per-layer calls (test_step_path.py:87-97)."""

import numpy as np
import pytest
import torch

import scripts as S
from echokv_amd.canary import canary_kl
from oracle import canary as OC

pytestmark = pytest.mark.gpu


def _close(got, ref, rtol=2e-3, atol=2e-6):
    got = got.cpu().numpy().astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=atol)


def test_canary_matches_reference_outputs(device):
    g = np.load(S.__file__.replace("scripts.py", "canary.npz"))
    (q, kref), (q2, kref2) = S.canary_inputs()
    got = canary_kl(torch.from_numpy(q).to(device), torch.from_numpy(kref).to(device), (2, 4, 8), 32, 64 ** -0.5)
    _close(got, g["small_out"])
    got2 = canary_kl(torch.from_numpy(q2).to(device), torch.from_numpy(kref2).to(device), (2, 4, 8), 16,
                     128 ** -0.5)
    _close(got2, g["cfg_out"])
    _close(got2, OC.canary_kl(q2.astype(np.float32), kref2, (2, 4, 8), 16, 128 ** -0.5))


def test_canary_batched_equals_per_layer_and_monotone(device):
    (q, kref), _ = S.canary_inputs()
    qd, kd = torch.from_numpy(q).to(device), torch.from_numpy(kref).to(device)
    batched = canary_kl(qd, kd, (2, 4, 8), 32, 64 ** -0.5)
    each = torch.stack([canary_kl(qd[i], kd[i], (2, 4, 8), 32, 64 ** -0.5) for i in range(3)])
    torch.testing.assert_close(batched, each, rtol=1e-6, atol=1e-7)
    d = batched.cpu().numpy()
    assert (d[:, 0] > d[:, 1]).all() and (d[:, 1] > d[:, 2]).all() and (d >= 0).all()
    low = canary_kl(qd.bfloat16(), kd, (2, 4, 8), 32, 64 ** -0.5)
    assert low.dtype == torch.float32 and low.shape == (3, 3)


@pytest.mark.parametrize("d", [72, 40])
def test_canary_head_size_not_multiple_of_16(device, d):
    """Query rows are read 16 channels at a time; the remaining channels of a
    head size that is not a multiple of 16 take the per-element tail."""
    rng = np.random.default_rng(d)
    q = rng.standard_normal((2, 4, 8, d)).astype(np.float32)     # [layers, nq, Hq, D]
    kref = rng.standard_normal((2, 48, 2, d)).astype(np.float32)  # [layers, W, H, D]
    got = canary_kl(torch.from_numpy(q).to(device), torch.from_numpy(kref).to(device), (2, 4, 8), 16, d ** -0.5)
    _close(got, OC.canary_kl(q, kref, (2, 4, 8), 16, d ** -0.5))


@pytest.mark.parametrize("window,kg,d,hq,h,nq", [
    (200, 16, 128, 32, 8, 8),    # three 64-key chunks and a partial one
    (100, 32, 128, 64, 8, 8),    # oldest 4 keys dropped; 64 query rows per workgroup
    (256, 128, 128, 8, 2, 4),    # K groups longer than a chunk: stats from memory
    (96, 16, 256, 16, 4, 2),     # head size 256: 32-key chunks
    (64, 64, 64, 4, 4, 8),       # one group, GQA 1
])
def test_canary_windows_beyond_one_chunk(device, window, kg, d, hq, h, nq):
    rng = np.random.default_rng(window + kg + d)
    layers = 3
    q = rng.standard_normal((layers, nq, hq, d)).astype(np.float32)
    kref = (rng.standard_normal((layers, window, h, d)) * 2).astype(np.float32)
    got = canary_kl(torch.from_numpy(q).to(device), torch.from_numpy(kref).to(device), (2, 4, 8), kg, d ** -0.5)
    ref = OC.canary_kl(q, kref, (2, 4, 8), kg, d ** -0.5)
    print(f"[canary W{window} KG{kg} D{d}] max rel err {float(np.abs(got.cpu().numpy() / ref - 1).max()):.2e}",
          flush=True)
    _close(got, ref)
    assert (ref[:, 0] > ref[:, 1]).all() and (ref[:, 1] > ref[:, 2]).all()
