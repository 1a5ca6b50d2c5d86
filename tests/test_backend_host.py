"""CPU: the plugin boundary without a GPU -- host slot mapping over fake vLLM
block tables (the scenarios of tests/echokv_vllm/test_host_slots.py:24-135),
the backend's answers to vLLM (backend.py:72-118), the implementation's
refusals (backend.py:499-524), the control API (control.py:39-117), the
reference's module path and entry point, and plugin registration gating."""

from dataclasses import dataclass, replace
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from echokv_amd import control, host_slots, plugin
from echokv_amd._vllm import AttentionCGSupport, MultipleOf
from echokv_amd.backend import CanaryClock, EchoKVAttentionBackend, EchoKVAttentionImpl, EchoKVMetadataBuilder
from echokv_amd.config import load_config
from echokv_amd.host_slots import host_lens_and_slots, install_v1, install_v1_dummy, install_v2, is_dummy_step
from echokv_amd.tiered_cache import TieredLayout

BS = 16


def device_slots(rows, qsl, seq, num_tokens):
    """vLLM's device slot mapping, computed token by token."""
    out = torch.full((num_tokens,), -1, dtype=torch.int64)
    for r in range(len(seq)):
        qs, qe = qsl[r], qsl[r + 1]
        for i, p in enumerate(range(seq[r] - (qe - qs), seq[r])):
            out[qs + i] = int(rows[r][p // BS]) * BS + p % BS
    return out


def cm_of(table, qsl, seq, num_tokens, req_idx=None):
    return SimpleNamespace(seq_lens_cpu_upper_bound=torch.tensor(seq, dtype=torch.int32), block_table_tensor=table,
                           num_reqs=len(seq), query_start_loc_cpu=torch.tensor(qsl, dtype=torch.int32),
                           num_actual_tokens=num_tokens, req_idx=req_idx)


class V2Tables:
    """What host_slots relies on of vLLM's V2 ``BlockTables``."""

    redirect_writes_to_null_block = False

    def __init__(self, max_reqs, max_blocks):
        self.num_kv_cache_groups = 1
        self.block_sizes = [BS]
        self.cp_size = 1
        self.block_tables = [SimpleNamespace(gpu=torch.zeros(max_reqs, max_blocks, dtype=torch.int32))]
        self.num_blocks = SimpleNamespace(np=np.zeros((1, max_reqs), dtype=np.int32))
        self.input_block_tables = [torch.zeros_like(self.block_tables[0].gpu)]

    def append_block_ids(self, req_index, new_block_ids, overwrite):
        start = 0 if overwrite else self.num_blocks.np[0, req_index]
        ids = new_block_ids[0]
        self.block_tables[0].gpu[req_index, start : start + len(ids)] = torch.tensor(ids, dtype=torch.int32)
        self.num_blocks.np[0, req_index] = start + len(ids)

    def compute_slot_mappings(self, *args):
        pass

    def get_dummy_slot_mappings(self, num_tokens):
        pass

    def gather(self, idx):
        self.input_block_tables[0][: len(idx)] = self.block_tables[0].gpu[idx]
        return self.input_block_tables[0][: len(idx)]


# ---- host_slots.py -----------------------------------------------------------------

def test_v2_mirror_follows_appends_and_slot_reuse():
    install_v2(V2Tables)
    install_v2(V2Tables)  # idempotent
    bt = V2Tables(4, 8)
    bt.append_block_ids(2, ([7, 3],), overwrite=True)
    bt.append_block_ids(0, ([5],), overwrite=True)
    bt.append_block_ids(2, ([11],), overwrite=False)  # the request in slot 2 grows
    bt.append_block_ids(0, ([9, 1],), overwrite=True)  # slot 0 reused by a new request
    req_idx = np.array([2, 0])  # batch row 0 = slot 2 decoding at 40, row 1 = slot 0 prefilling 20
    table = bt.gather(torch.tensor(req_idx))
    qsl, seq, t = [0, 1, 21, 21], [41, 20, 0], 24
    lens, slots = host_lens_and_slots(cm_of(table, qsl, seq, t, req_idx), BS)
    assert lens.tolist() == seq
    assert torch.equal(slots, device_slots([[7, 3, 11], [9, 1], []], qsl, seq, t))


def test_unknown_tables_and_block_sizes_fall_back_to_the_device_copy():
    install_v2(V2Tables)
    bt = V2Tables(2, 4)
    bt.append_block_ids(0, ([1],), overwrite=True)
    table = bt.gather(torch.tensor([0]))
    cm = cm_of(table, [0, 1], [3], 1, np.array([0]))
    assert host_lens_and_slots(cm, BS * 2) is None
    assert host_lens_and_slots(cm_of(torch.zeros(1, 4), [0, 1], [3], 1), BS) is None
    cm.seq_lens_cpu_upper_bound = None
    assert host_lens_and_slots(cm, BS) is None
    cm = cm_of(table, [0, 1], [3], 1, None)  # V2 without req_idx
    assert host_lens_and_slots(cm, BS) is None


def test_v1_tables_are_indexed_by_batch_row(monkeypatch):
    np_table = np.array([[4, 6, 0, 0], [2, 0, 0, 0], [0] * 4])
    monkeypatch.setattr(host_slots, "_host_table", lambda cm, bs: (np_table, None))
    qsl, seq = [0, 3, 4], [20, 9]
    _, slots = host_lens_and_slots(cm_of(torch.zeros(3, 4), qsl, seq, 4), BS)
    assert torch.equal(slots, device_slots(np_table, qsl, seq, 4))


def test_v1_registry_lookup_and_dummy_depth():
    class Table:
        def __init__(self):
            self.block_size, self.dcp_world_size, self.pcp_world_size = BS, 1, 1
            self.block_table = SimpleNamespace(gpu=torch.zeros(2, 4, dtype=torch.int32),
                                               np=np.array([[3, 8, 0, 0], [5, 0, 0, 0]]))

    install_v1(Table)
    install_v1(Table)  # idempotent
    t = Table()
    cm = cm_of(t.block_table.gpu, [0, 1, 3], [18, 2], 3)
    _, slots = host_lens_and_slots(cm, BS)
    assert torch.equal(slots, device_slots(t.block_table.np, [0, 1, 3], [18, 2], 3))
    assert not is_dummy_step(cm)

    class Runner:
        def _dummy_run(self, probe):
            return probe()

    install_v1_dummy(Runner)
    assert Runner()._dummy_run(lambda: (is_dummy_step(cm), host_lens_and_slots(cm, BS))) == (True, None)
    assert host_slots.REGISTRY.v1_dummy_runs == 0


def test_v2_dummy_steps_use_the_device_copy():
    install_v2(V2Tables)
    bt = V2Tables(2, 4)
    bt.append_block_ids(0, ([3],), overwrite=True)
    cm = cm_of(bt.gather(torch.tensor([0])), [0, 1], [5], 1, np.array([0]))
    bt.compute_slot_mappings()
    assert host_lens_and_slots(cm, BS) is not None and not is_dummy_step(cm)
    bt.get_dummy_slot_mappings(1)
    assert host_lens_and_slots(cm, BS) is None and is_dummy_step(cm)
    bt.compute_slot_mappings()
    assert host_lens_and_slots(cm, BS) is not None


# ---- backend.py ----------------------------------------------------------------------

@dataclass(frozen=True)
class Spec:
    block_size: int = 32
    num_kv_heads: int = 8
    head_size: int = 128
    head_size_v: int = 128
    dtype: torch.dtype = torch.bfloat16
    num_head_slots: int = 8
    state_content_bytes: int = 0


def test_backend_answers(monkeypatch):
    for v in ("ECHOKV_MEM_BITS", "ECHOKV_K_GROUP", "ECHOKV_V_GROUP", "ECHOKV_CUDAGRAPH"):
        monkeypatch.delenv(v, raising=False)
    B = EchoKVAttentionBackend
    assert B.get_name() == "CUSTOM" and not B.forward_includes_kv_cache_update
    spec = B.customize_spec(Spec())
    assert spec.num_head_slots == 1
    assert spec.state_content_bytes == TieredLayout.per_token_bytes(8, 128, 4, 32, 32)
    with pytest.raises(NotImplementedError):
        B.customize_spec(replace(Spec(), head_size_v=64))
    assert B.get_supported_kernel_block_sizes() == [MultipleOf(32)]
    assert B.supports_block_size(64) and not B.supports_block_size(16) and B.supports_block_size(None)
    monkeypatch.setenv("ECHOKV_K_GROUP", "16")
    assert B.supports_block_size(16) and B.get_supported_kernel_block_sizes() == [MultipleOf(16)]
    # The reference's rule (a multiple of 4 and of the V group), up to 256 channels.
    assert B.supports_head_size(128) and B.supports_head_size(64) and B.supports_head_size(96)
    assert B.supports_head_size(256) and not B.supports_head_size(80) and not B.supports_head_size(512)
    assert B.supports_attn_type("decoder") and not B.supports_attn_type("encoder")
    assert B.get_impl_cls() is EchoKVAttentionImpl and B.get_builder_cls() is EchoKVMetadataBuilder
    assert EchoKVMetadataBuilder.get_cudagraph_support(None, Spec()) == AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE
    assert EchoKVMetadataBuilder.get_cudagraph_support(None, Spec(block_size=48)) == AttentionCGSupport.NEVER
    monkeypatch.setenv("ECHOKV_CUDAGRAPH", "0")
    assert EchoKVMetadataBuilder.get_cudagraph_support(None, Spec()) == AttentionCGSupport.NEVER


@pytest.mark.parametrize("kw,what", [({"alibi_slopes": [1.0]}, "alibi"), ({"sliding_window": 128}, "sliding window"),
                                     ({"logits_soft_cap": 30.0}, "soft cap"), ({"sinks": torch.zeros(1)}, "sinks"),
                                     ({"kv_sharing_target_layer_name": "x"}, "KV sharing"),
                                     ({"attn_type": "encoder"}, "attn_type")])
def test_impl_refuses_unsupported_features(kw, what):
    with pytest.raises(NotImplementedError, match=what):
        EchoKVAttentionImpl(32, 128, 0.088, 8, **kw)


def test_own_group_exact_needs_the_mfma_prefill_layouts(monkeypatch):
    monkeypatch.setenv("ECHOKV_OWN_GROUP_EXACT", "1")
    monkeypatch.setenv("ECHOKV_K_GROUP", "16")
    EchoKVAttentionImpl(32, 128, 0.088, 8)
    with pytest.raises(NotImplementedError, match="OWN_GROUP_EXACT"):
        EchoKVAttentionImpl(32, 96, 0.088, 8)


def test_impl_buffers_follow_the_config(monkeypatch):
    monkeypatch.setenv("ECHOKV_K_GROUP", "16")
    monkeypatch.setenv("ECHOKV_RESIDUAL_SLOTS", "20")
    monkeypatch.setenv("ECHOKV_KREF_WINDOW", "48")
    impl = EchoKVAttentionImpl(32, 128, 0.088, 8)
    assert tuple(impl.residual.shape) == (21, 16, 8, 128)
    assert tuple(impl.kref_buf.shape) == (48, 8, 128) and impl.kref_buf.dtype == torch.float32
    assert tuple(impl.stash.shape) == (8, 32, 128)
    assert impl.store is None and impl.controller.bits == 4


# ---- control.py ----------------------------------------------------------------------

class Attn(torch.nn.Module):
    def __init__(self, name):
        super().__init__()
        self.layer_name = name
        self.impl = EchoKVAttentionImpl(4, 64, 0.125, 2)


class Model(torch.nn.Module):
    def __init__(self, n):
        super().__init__()
        # registered out of order: iter_layers sorts by the layer number in the name
        self.attn = torch.nn.ModuleList([Attn(f"model.layers.{i}.self_attn.attn") for i in reversed(range(n))])


def test_control_api_steers_every_layer():
    m = Model(3)
    assert [n for n, _ in control.iter_layers(m)] == [f"model.layers.{i}.self_attn.attn" for i in range(3)]
    assert control.set_tier_vector(m, [8, 2, 4]) == 3
    assert control.get_tier_vector(m) == [8, 2, 4]
    assert control.set_tier_vector(m, 2) == 3 and control.get_tier_vector(m) == [2, 2, 2]
    with pytest.raises(ValueError):
        control.set_tier_vector(m, [4, 4])
    with pytest.raises(ValueError):
        control.set_tier_vector(m, [4, 4, 3])
    control.set_frozen(m, True)
    control.set_tau0(m, 0.05)
    impl = control.iter_layers(m)[0][1]
    assert impl.controller.params.frozen and impl.controller.params.tau0 == 0.05
    impl.controller.observe({2: 1.0, 4: 1.0, 8: 1.0}, ctx_len=10)
    assert impl.controller.bits == 2  # frozen
    st = control.get_state(m)
    assert st["tier_vector"] == [2, 2, 2] and st["avg_stored_bits"] is None
    assert st["layers"][0]["fires"] == 1 and st["layers"][0]["ema"]["2"] == 1.0
    impl.forward_calls = 5
    assert control.reset_counters(m) == 3 and impl.forward_calls == 0


# ---- canary schedule --------------------------------------------------------------

def test_canary_clock_fires_on_the_interval_and_waits_for_a_live_request():
    clock = CanaryClock(interval=3)
    armed = [clock.tick(dummy=False) for _ in range(3)]
    assert armed == [False, False, True]
    clock.fired(0, 0.0)  # no live request on the armed step: stays armed
    assert clock.tick(dummy=True) and clock.steps == 3  # dummy steps do not count
    clock.fired(2, 100.0)
    assert not clock.armed and clock.stashed == (2, 100.0)
    assert [clock.tick(dummy=False) for _ in range(3)] == [False, False, True]


# ---- the reference's module path -------------------------------------------------------

def test_reference_module_path_is_this_package():
    import importlib

    import echokv_amd.backend
    import echokv_amd.kernels.decode
    from echokv_vllm import control as ref_control
    from echokv_vllm.kernels import decode as ref_decode

    assert ref_control is control and ref_decode is echokv_amd.kernels.decode
    mod, cls = plugin.BACKEND_PATH.rsplit(".", 1)
    assert mod == "echokv_vllm.backend" and importlib.import_module(mod) is echokv_amd.backend
    assert getattr(importlib.import_module(mod), cls) is EchoKVAttentionBackend
    try:
        import tomllib
    except ImportError:  # Python 3.10
        import tomli as tomllib
    from pathlib import Path

    meta = tomllib.loads((Path(__file__).resolve().parents[1] / "pyproject.toml").read_text())
    assert meta["project"]["entry-points"]["vllm.general_plugins"] == {"echokv": "echokv_vllm.plugin:register"}


# ---- V groups ----------------------------------------------------------------------------

def test_any_v_group_dividing_the_head_size_is_taken(monkeypatch):
    """The reference's rule (``backend.py:100-102``): the head size must divide by
    the V group (and by 4); any such V group is stored, powers of two or not."""
    for vg, ok96 in (("4", True), ("16", True), ("24", True), ("6", True), ("3", True), ("1", True),
                     ("64", False), ("20", False)):
        monkeypatch.setenv("ECHOKV_V_GROUP", vg)
        assert load_config().v_group == int(vg)
        assert EchoKVAttentionBackend.supports_head_size(96) is ok96
    monkeypatch.setenv("ECHOKV_V_GROUP", "20")
    assert EchoKVAttentionBackend.supports_head_size(80)
    for vg in ("0", "512"):
        monkeypatch.setenv("ECHOKV_V_GROUP", vg)
        with pytest.raises(ValueError, match="ECHOKV_V_GROUP"):
            load_config()


def test_batch_invariant_is_the_default_and_can_be_turned_off(monkeypatch):
    monkeypatch.delenv("ECHOKV_BATCH_INVARIANT", raising=False)
    assert load_config().batch_invariant
    monkeypatch.setenv("ECHOKV_BATCH_INVARIANT", "0")
    assert not load_config().batch_invariant


def test_register_is_gated_by_echokv_enable(monkeypatch):
    monkeypatch.delenv("ECHOKV_ENABLE", raising=False)
    plugin.register()  # disabled: returns before importing vLLM
    assert plugin.BACKEND_PATH == "echokv_vllm.backend.EchoKVAttentionBackend"
