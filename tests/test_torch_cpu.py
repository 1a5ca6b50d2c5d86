"""CPU: pin the torch CPU restatement (``oracle/torch_cpu.py``, the benchmark's CPU
baseline) to the reference's own outputs: quantization bytes (``quant.npz``),
whole page bytes after every golden write script with the torch write path in
place of the oracle's, the reference's decode / prefill outputs on the config-1
stores and its canary outputs."""

import hashlib

import numpy as np
import pytest
import torch

import scripts as S
from host_sim import SimStore, golden, replay
from oracle import torch_cpu as TC

QG = np.load(S.__file__.replace("scripts.py", "quant.npz"), allow_pickle=False)
CG = np.load(S.__file__.replace("scripts.py", "canary.npz"), allow_pickle=False)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_and_pack_match_reference_bytes(bits):
    xs, k = S.quant_inputs()
    for shift, x in xs.items():
        tag = f"s{int(shift)}_b{bits}"
        c, sc, mn = TC.quantize(torch.from_numpy(x), bits, 32)
        assert np.array_equal(c.numpy(), QG[f"codes_{tag}"])
        assert np.array_equal(sc.numpy().view(np.uint16), QG[f"scale_{tag}"].view(np.uint16))
        assert np.array_equal(mn.numpy().view(np.uint16), QG[f"min_{tag}"].view(np.uint16))
        assert np.array_equal(TC.pack(c, bits).numpy(), QG[f"packed_{tag}"])
        assert torch.equal(TC.unpack(TC.pack(c, bits), bits), c)
    sc, mn = TC.stats_along(torch.from_numpy(k[:32]), bits, 0)
    assert np.array_equal(sc.numpy().view(np.uint16), QG[f"stats_scale_b{bits}"].view(np.uint16))
    assert np.array_equal(TC.fake_quant_channels(torch.from_numpy(k), bits, 32).numpy(), QG[f"fqc_b{bits}"])


class TorchWrites(SimStore):
    """The replay of ``host_sim`` with the torch write path doing the step's writes."""

    def __init__(self, s):
        super().__init__(s)
        ps = self.ps
        kref = lambda: None if self.kref is None else torch.from_numpy(self.kref)  # noqa: E731
        ps.finalize_k = lambda k, fin: TC.finalize_k(ps, torch.from_numpy(k), fin)
        ps.write_tokens = lambda k, v, tok, _kr: TC.write_tokens(ps, torch.from_numpy(k), torch.from_numpy(v), tok,
                                                                 kref())


@pytest.mark.parametrize("name", [s.name for s in S.all_scripts()])
def test_torch_write_path_reproduces_reference_bytes(name):
    s = next(x for x in S.all_scripts() if x.name == name)
    g = golden(name)
    sim = TorchWrites(s)
    for slots, bits, k, v in S.script_inputs(s):
        sim.write(k, v, slots, bits)
    pages = sim.ps.pages
    if s.full_bytes:
        assert np.array_equal(pages, g["pages"])
    else:
        got = np.array([hashlib.sha256(pages[b].tobytes()).hexdigest() for b in range(s.num_blocks)])
        assert np.array_equal(got, g["page_sha"])
    live = sim.ps.block_res[sim.ps.block_res >= 0]
    assert np.array_equal(sim.ps.res_k[live], g["res_live"])
    if sim.kref is not None:
        assert np.array_equal(sim.kref, g["kref"])


@pytest.fixture(scope="module")
def cfg1():
    return {n: replay(next(s for s in S.all_scripts() if s.name == n))
            for n in ("cfg1_int8_bs16", "cfg1_int4_bs16", "cfg1_int2_bs16", "cfg1_int4_bs32")}


@pytest.mark.parametrize("name", ["cfg1_int8_bs16", "cfg1_int4_bs16", "cfg1_int2_bs16", "cfg1_int4_bs32"])
def test_torch_decode_matches_reference_output(cfg1, name):
    sim = cfg1[name]
    s = sim.s
    q = torch.from_numpy(S.cfg1_query(s).astype(np.float32))
    out = TC.decode(sim.ps, q, s.meta["table"], s.meta["lens"], s.d ** -0.5)
    assert np.abs(out.numpy() - golden(name)["decode_out"]).max() < 2e-5


def test_torch_gather_and_prefill_match_reference_output(cfg1):
    sim = cfg1["cfg1_int4_bs16"]
    s, g = sim.s, golden("cfg1_int4_bs16")
    P = TC.Pages(sim.ps)
    pos = torch.arange(64)
    k, v = TC.gather(P, torch.as_tensor(s.meta["table"][0])[pos // s.bs], pos % s.bs)
    assert np.array_equal(k.numpy(), g["gather0_k"]) and np.array_equal(v.numpy(), g["gather0_v"])
    prefill, req_of, pq = S.cfg1_prefill(s)
    out = TC.prefill(sim.ps, torch.from_numpy(pq.astype(np.float32)), prefill, req_of, s.meta["table"], s.d ** -0.5)
    assert np.abs(out.numpy() - g["prefill_out"]).max() < 2e-5


def test_torch_canary_matches_reference_outputs():
    (q, kref), (q2, kref2) = S.canary_inputs()
    a = TC.canary_kl(torch.from_numpy(q), torch.from_numpy(kref), (2, 4, 8), 32, 64 ** -0.5).numpy()
    b = TC.canary_kl(torch.from_numpy(q2), torch.from_numpy(kref2), (2, 4, 8), 16, 128 ** -0.5).numpy()
    assert np.allclose(a, CG["small_out"], rtol=2e-3, atol=1e-6)
    assert np.allclose(b, CG["cfg_out"], rtol=2e-3, atol=1e-6)
