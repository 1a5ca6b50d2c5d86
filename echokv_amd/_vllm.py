"""The parts of vLLM's attention-backend interface the EchoKV backend uses.

With vLLM installed these are vLLM's own classes and functions (the names the
reference backend imports, ``echokv_vllm/backend.py:37-49``). Without it -- this
build's test machines, where the backend is driven by fake vLLM objects as the
reference's own host-slot tests do -- they are minimal stand-ins with the same
names and constructor arguments; nothing here computes anything.
"""

from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Generic, TypeVar

try:  # vLLM 0.32 layout
    from vllm.forward_context import get_forward_context as _vllm_forward_context
    from vllm.v1.attention.backend import (  # noqa: F401
        AttentionBackend,
        AttentionCGSupport,
        AttentionImpl,
        AttentionLayer,
        AttentionMetadataBuilder,
        AttentionType,
        CommonAttentionMetadata,
        MultipleOf,
    )

    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False
    _vllm_forward_context = None
    M = TypeVar("M")

    class AttentionBackend:
        """Stand-in for vllm.v1.attention.backend.AttentionBackend."""

    class AttentionImpl(Generic[M]):
        """Stand-in for vllm.v1.attention.backend.AttentionImpl."""

    class AttentionLayer:
        """Stand-in for vllm.v1.attention.backend.AttentionLayer."""

    class CommonAttentionMetadata:
        """Stand-in for vllm.v1.attention.backend.CommonAttentionMetadata."""

    class AttentionMetadataBuilder(Generic[M]):
        """Stand-in for vllm.v1.attention.backend.AttentionMetadataBuilder."""

        def __init__(self, kv_cache_spec, layer_names, vllm_config, device) -> None:
            self.kv_cache_spec = kv_cache_spec
            self.layer_names = layer_names
            self.vllm_config = vllm_config
            self.device = device

    class AttentionCGSupport(enum.Enum):
        NEVER = 0
        UNIFORM_SINGLE_TOKEN_DECODE = 1
        UNIFORM_BATCH = 2
        ALWAYS = 3

    class AttentionType:
        DECODER = "decoder"
        ENCODER = "encoder"
        ENCODER_ONLY = "encoder_only"
        ENCODER_DECODER = "encoder_decoder"

    @dataclass(frozen=True)
    class MultipleOf:
        base: int


# Metadata for callers that drive the backend without vLLM's forward context
# (the tests, standalone drivers): set_forward_metadata(md) before the layers run.
_local_metadata = None


def set_forward_metadata(md) -> None:
    global _local_metadata
    _local_metadata = md


def forward_metadata():
    """The current step's attention metadata (vLLM's forward context when it runs the model)."""
    if _vllm_forward_context is not None:
        try:
            return _vllm_forward_context().attn_metadata
        except (AssertionError, AttributeError):  # no forward context set: a standalone driver
            pass
    return _local_metadata


def num_attention_heads(vllm_config, layer_names) -> int:
    if HAVE_VLLM:
        from vllm.v1.attention.backends.utils import get_num_attention_heads_from_layers

        n = get_num_attention_heads_from_layers(vllm_config, layer_names)
        if n:
            return n
    return vllm_config.model_config.get_num_attention_heads(vllm_config.parallel_config)


def attention_layers(vllm_config, layer_names) -> list:
    from vllm.config import get_layers_from_vllm_config
    from vllm.model_executor.layers.attention_layer_base import AttentionLayerBase

    return list(get_layers_from_vllm_config(vllm_config, AttentionLayerBase, layer_names).values())


def current_vllm_config():
    if not HAVE_VLLM:
        return None
    from vllm.config import get_current_vllm_config_or_none

    return get_current_vllm_config_or_none()


def tp_mean(x):
    """Mean over tensor-parallel ranks (each rank's canary sees only its own KV heads)."""
    if not HAVE_VLLM:
        return x
    from vllm.distributed import get_tensor_model_parallel_world_size, tensor_model_parallel_all_reduce

    world = get_tensor_model_parallel_world_size()
    return x if world == 1 else tensor_model_parallel_all_reduce(x) / world
