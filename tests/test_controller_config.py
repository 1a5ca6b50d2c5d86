"""CPU: the tier controller, the ECHOKV_* settings and the K_ref ring, on the
known answers of tests/echokv_vllm/test_canary_controller.py:20-108 and
test_step_path.py:87-97, plus the closed forms they rest on."""

import math

import pytest
import torch

from echokv_amd.canary import KRefRing, ring_view
from echokv_amd.config import SETTINGS, default_init_bits, load_config
from echokv_amd.controller import ControllerParams, LayerController


def make(**kw):
    return LayerController(ControllerParams(**kw))


# ---- controller.py:45-68 -----------------------------------------------------------

def test_lowest_tier_under_budget_else_highest():
    c = make(tau0=0.01, l0=4096, alpha=1.0, init_bits=8)
    c.observe({2: 0.5, 4: 0.005, 8: 0.0001}, ctx_len=4096)
    assert c.bits == 4
    c.observe({2: 0.001, 4: 0.0005, 8: 0.0001}, ctx_len=4096)
    assert c.bits == 2
    c.observe({2: 0.5, 4: 0.5, 8: 0.5}, ctx_len=4096)
    assert c.bits == 8  # nothing under budget: the highest tier
    assert c.transitions == 3 and c.fires == 3


def test_ema_weights_the_newest_sample_by_alpha():
    c = make(alpha=0.25, init_bits=8)
    c.observe({2: 1.0, 4: 0.0, 8: 0.0}, ctx_len=1)
    assert c.ema[2] == 1.0  # the first sample is taken as is
    c.observe({2: 0.0, 4: 0.0, 8: 0.0}, ctx_len=1)
    assert c.ema[2] == pytest.approx(0.75)
    c.observe({2: 1.0, 4: 0.0, 8: 0.0}, ctx_len=1)
    assert c.ema[2] == pytest.approx(0.25 + 0.75 * 0.75)


def test_tau_sqrt_scaling_only_loosens():
    c = make(tau0=0.022, l0=4096, tau_scaling="sqrt")
    assert math.isclose(c.tau(4096 * 32), 0.022 * math.sqrt(32))
    assert c.tau(100) == 0.022  # short contexts never tighten it
    assert make(tau0=0.022).tau(4096 * 32) == 0.022  # no scaling by default
    c = make(tau0=0.01, l0=4096, alpha=1.0, tau_scaling="sqrt")
    c.observe({2: 0.03, 4: 0.001, 8: 0.0}, ctx_len=4096)
    assert c.bits == 4
    c.observe({2: 0.03, 4: 0.001, 8: 0.0}, ctx_len=4096 * 16)  # tau = 0.04
    assert c.bits == 2


def test_frozen_and_fixed_hold_the_tier_but_track_the_ema():
    c = make(alpha=0.5, init_bits=8, frozen=True)
    c.observe({2: 0.0, 4: 0.0, 8: 0.0}, ctx_len=100)
    c.observe({2: 1.0, 4: 1.0, 8: 1.0}, ctx_len=100)
    assert c.bits == 8 and c.ema[2] == 0.5 and c.transitions == 0
    c = make(fixed_bits=2)
    c.observe({2: 9.0, 4: 9.0, 8: 9.0}, ctx_len=100)
    assert c.bits == 2


# ---- config.py:40-99 -----------------------------------------------------------------

def test_defaults_and_budget_rules():
    cfg = load_config({})
    assert (cfg.mem_bits, cfg.controller.init_bits, cfg.k_group, cfg.v_group) == (4, 4, 32, 32)
    assert (cfg.canary_interval, cfg.kref_window, cfg.canary_max_q, cfg.residual_slots) == (64, 64, 8, None)
    assert (cfg.controller.tau0, cfg.controller.alpha, cfg.controller.l0) == (0.01, 0.1, 4096)
    assert load_config({"ECHOKV_FIXED_BITS": "8"}).mem_bits == 8  # a pinned tier gets its budget
    assert load_config({"ECHOKV_FIXED_BITS": "2"}).mem_bits == 2
    assert load_config({"ECHOKV_MEM_BITS": "6"}).controller.init_bits == 4
    assert load_config({"ECHOKV_MEM_BITS": "8"}).controller.init_bits == 8
    assert [default_init_bits(m) for m in (2, 4, 6, 8)] == [2, 4, 4, 8]
    assert load_config({"ECHOKV_FROZEN": "1"}).controller.frozen
    assert load_config({"ECHOKV_MEM_BITS": ""}).mem_bits == 4  # empty = unset
    assert not cfg.own_group_exact and load_config({"ECHOKV_OWN_GROUP_EXACT": "1"}).own_group_exact


def test_environment_is_read(monkeypatch):
    for var in ("ECHOKV_MEM_BITS", "ECHOKV_INIT_BITS", "ECHOKV_FIXED_BITS", "ECHOKV_K_GROUP"):
        monkeypatch.delenv(var, raising=False)
    monkeypatch.setenv("ECHOKV_K_GROUP", "16")
    monkeypatch.setenv("ECHOKV_KREF_WINDOW", "200")
    cfg = load_config()
    assert cfg.k_group == 16 and cfg.kref_window == 200


@pytest.mark.parametrize("env,name", [
    ({"ECHOKV_K_GROUP": "8"}, "ECHOKV_K_GROUP"),
    ({"ECHOKV_K_GROUP": "48"}, "ECHOKV_K_GROUP"),
    ({"ECHOKV_MEM_BITS": "5"}, "ECHOKV_MEM_BITS"),
    ({"ECHOKV_INIT_BITS": "3"}, "ECHOKV_INIT_BITS"),
    ({"ECHOKV_FIXED_BITS": "16"}, "ECHOKV_FIXED_BITS"),
    ({"ECHOKV_TAU_SCALING": "log"}, "ECHOKV_TAU_SCALING"),
    ({"ECHOKV_CANARY_INTERVAL": "0"}, "ECHOKV_CANARY_INTERVAL"),
    ({"ECHOKV_KREF_WINDOW": "16"}, "ECHOKV_KREF_WINDOW"),  # below the default K group of 32
    ({"ECHOKV_OWN_GROUP_EXACT": "1", "ECHOKV_K_GROUP": "128", "ECHOKV_KREF_WINDOW": "128"}, "ECHOKV_OWN_GROUP_EXACT"),
])
def test_bad_values_raise_value_error_naming_the_variable(env, name):
    with pytest.raises(ValueError, match=name):
        load_config(env)


def test_every_variable_has_one_row():
    envs = [s.env for s in SETTINGS]
    assert len(envs) == len(set(envs)) == 16


# ---- canary.py:19-56 -----------------------------------------------------------------

def test_kref_ring_keeps_the_last_window_oldest_first():
    ring = KRefRing(4)
    assert ring.view() is None
    ring.push(torch.arange(3).float().view(3, 1, 1))
    assert ring.view().flatten().tolist() == [0.0, 1.0, 2.0]
    ring.push(torch.arange(3, 9).float().view(6, 1, 1))
    assert ring.view().flatten().tolist() == [5.0, 6.0, 7.0, 8.0]
    ring.push(torch.tensor([9.0]).view(1, 1, 1))
    assert ring.view().flatten().tolist() == [6.0, 7.0, 8.0, 9.0]
    ring.push(torch.zeros(0, 1, 1))
    assert ring.view().flatten().tolist() == [6.0, 7.0, 8.0, 9.0]


def test_ring_view_along_a_layer_stack():
    """The backend stacks every layer's ring and views dim 1 (backend.py:330)."""
    buf = torch.arange(2 * 5).float().view(2, 5, 1)
    assert ring_view(buf, 3, 5, dim=1)[0].flatten().tolist() == [3.0, 4.0, 0.0, 1.0, 2.0]
    assert ring_view(buf, 3, 3, dim=1)[1].flatten().tolist() == [5.0, 6.0, 7.0]  # never wrapped
    assert ring_view(buf, 1, 3, dim=1)[0].flatten().tolist() == [3.0, 4.0, 0.0]  # wrapped, not full
    with pytest.raises(ValueError):
        ring_view(buf, 0, 6, dim=1)
