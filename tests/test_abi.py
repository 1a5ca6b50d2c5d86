"""CPU: the C-ABI library loads and exports every entry point ``include/echokv.h``
declares, and its host-side argument checks reject bad input before any launch
(no GPU needed: nothing below reaches a kernel)."""

import ctypes as C
import re
from pathlib import Path

import pytest

from echokv_amd import _lib
from echokv_amd.tiered_cache import TieredLayout

HEADER = Path(__file__).resolve().parents[1] / "include" / "echokv.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(echokv_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built: run python -c 'import __graft_entry__ as g; g.build()'")
    return _lib.lib()


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.EXPORTS)
    assert set(_lib._SIGS) == set(names) - {"echokv_error_string", "echokv_prefill_dense_workspace",
                                            "echokv_decode_workspace_rows"}


def test_decode_workspace_rows_of_the_split_schedule(lib):
    # The split schedule needs no device query: num_seqs * num_splits rows.
    L = _layout()
    assert lib.echokv_decode_workspace_rows(C.byref(L), 32, _lib.F16, 7, 5, _lib.DECODE_BATCH_INVARIANT) == 35
    assert lib.echokv_decode_workspace_rows(C.byref(L), 32, _lib.F16, 0, 5, 0) == 0
    assert lib.echokv_decode_workspace_rows(C.byref(L), 30, _lib.F16, 7, 5, 1) == -1  # GQA not whole
    assert lib.echokv_decode_workspace_rows(C.byref(L), 32, 9, 7, 5, 1) == -1  # dtype
    assert lib.echokv_decode_workspace_rows(C.byref(L), 32, _lib.F16, 7, 0, 1) == -1  # no splits


def test_error_strings(lib):
    for code in range(5):
        assert lib.echokv_error_string(code)
    assert lib.echokv_error_string(0) != lib.echokv_error_string(1)


def _layout(**kw):
    lay = TieredLayout(8, 128, 16, 8, 16, 32)
    L = lay.abi(100, lay.page_bytes)
    for k, v in kw.items():
        setattr(L, k, v)
    return L


def _decode(lib, L, tier=4, splits=4, seqs=1, flags=0, tier_mask=None):
    res = _lib.Residual(C.c_void_p(16), 1, 2, 16 * 8 * 128, 8 * 128, 128)
    p = C.c_void_p(64)  # never dereferenced: every call below fails its checks first
    return lib.echokv_decode(C.byref(L), p, p, p, C.byref(res), p, 4096, 128, 1, 32, None, p, 64, None, p, seqs,
                             0.088, splits, 16, tier, tier_mask, flags, p, p, p, 4096, 128, 1, None)


def _layout_of(head_size=128, block_size=16, k_group=16, v_group=32):
    lay = TieredLayout(8, head_size, block_size, 8, k_group, v_group)
    return lay.abi(100, lay.page_bytes)


def test_decode_rejects_bad_arguments_before_launching(lib):
    assert _decode(lib, _layout_of(head_size=512)) == 2     # above the fp32 kernel's 256 channels
    assert _decode(lib, _layout(head_size=96)) == 2          # chunk bytes do not match the head size
    assert _decode(lib, _layout(block_size=24)) == 2         # block not a multiple of 16
    # Layouts the MFMA kernels are not built for pass the checks (the fp32 kernel takes them).
    for L in (_layout_of(head_size=96), _layout_of(head_size=256), _layout_of(block_size=48), _layout_of(k_group=8)):
        assert _decode(lib, L, seqs=0) == 0
    assert _decode(lib, _layout(), tier=3) != 0
    assert _decode(lib, _layout(), splits=0) != 0
    assert _decode(lib, _layout(), seqs=-1) != 0
    assert _decode(lib, _layout(), flags=2) != 0              # unknown schedule flag
    # Tier passes continue partial rows: the split schedule only.
    assert _decode(lib, _layout(), seqs=0, tier_mask=C.c_void_p(64)) == 1
    assert _decode(lib, _layout(), seqs=0, tier_mask=C.c_void_p(64), flags=_lib.DECODE_BATCH_INVARIANT) == 0
    assert _decode(lib, _layout(), seqs=0) == 0              # nothing to do: no launch


def test_store_entry_points_reject_bad_layouts(lib):
    L = _layout(chunk_bytes=12345)
    p = C.c_void_p(64)
    res = _lib.Residual(C.c_void_p(16), 1, 2, 16 * 8 * 128, 8 * 128, 128)
    rc = lib.echokv_write_tokens(C.byref(L), p, p, 1024, 128, p, 1024, 128, 1, p, 64, 4, C.byref(res), None, 0, 0,
                                 None)
    assert rc == 2
    rc = lib.echokv_store_blocks(C.byref(_layout()), p, p, 1, p, p, 3, None)
    assert rc != 0  # bits must be 2, 4 or 8


def _prefill_dense(lib, L, hq=32, tile_m=64, n_packs=4, n_q=2, ws_bytes=None, own_group=0):
    res = _lib.Residual(C.c_void_p(16), 1, 2, 16 * 8 * 128, 8 * 128, 128)
    p = C.c_void_p(64)  # never dereferenced: every call below fails its checks first
    if ws_bytes is None:
        ws_bytes = lib.echokv_prefill_dense_workspace(C.byref(L), n_packs)
    return lib.echokv_prefill_dense(C.byref(L), p, p, p, C.byref(res), p, 4096, 128, 1, hq, p, 4096, 128, 1, p,
                                    n_packs, p, n_q, tile_m, p, 64, p, ws_bytes, 0.088, own_group, None, None)


def _prefill(lib, L, hq=32, tile_m=32, n_tiles=0, own_group=0):
    res = _lib.Residual(C.c_void_p(16), 1, 2, 16 * 8 * 128, 8 * 128, 128)
    p = C.c_void_p(64)  # never dereferenced: every call below fails its checks first or launches nothing
    return lib.echokv_prefill(C.byref(L), p, p, p, C.byref(res), p, 4096, 128, 1, hq, p, 4096, 128, 1, p, n_tiles,
                              tile_m, p, 64, 0.088, own_group, None, None)


def test_prefill_tile_sizes_by_kernel(lib):
    """MFMA tiles hold 128 / GQA tokens (64 / GQA at head size 256); other layouts
    (fp32 kernel) 16 / GQA, no own group."""
    assert _prefill(lib, _layout_of(), tile_m=32) == 0                    # D 128, GQA 4: 128 / 4
    assert _prefill(lib, _layout_of(), tile_m=4) == 2
    assert _prefill(lib, _layout_of(head_size=256), tile_m=16) == 0       # D 256, GQA 4: 64 / 4
    assert _prefill(lib, _layout_of(head_size=256), tile_m=32) == 2
    assert _prefill(lib, _layout_of(head_size=256), hq=8 * 20, tile_m=3) == 0  # GQA 20: 64 // 20
    assert _prefill(lib, _layout_of(head_size=256), hq=8 * 80, tile_m=1) == 0  # GQA 80 > 64: fp32 kernel
    assert _prefill(lib, _layout_of(head_size=96), tile_m=4) == 0         # fp32 kernel: 16 / 4
    assert _prefill(lib, _layout_of(head_size=96), tile_m=32) == 2
    assert _prefill(lib, _layout_of(head_size=96), tile_m=4, own_group=1) == 2
    assert _prefill(lib, _layout_of(head_size=512), tile_m=4) == 2


def _own_group(lib, L, hq=32, n=2):
    res = _lib.Residual(C.c_void_p(16), 1, 2, 16 * 8 * 128, 8 * 128, 128)
    p = C.c_void_p(64)  # never dereferenced: every call below fails its checks first
    return lib.echokv_prefill_own_group(C.byref(L), p, p, p, C.byref(res), p, 4096, 128, 1, hq, p, 1024, 128, 1,
                                        p, n, p, 64, p, 4096, 128, p, p, 4096, 128, 1, 0.088, None)


def test_own_group_prefill_argument_checks(lib):
    L = _layout()
    assert _prefill_dense(lib, L, own_group=2) == 1            # own_group is 0 or 1
    assert _own_group(lib, _layout(head_size=256)) == 2        # head_size <= 128
    assert _own_group(lib, L, hq=8 * 32) == 2                  # GQA <= 16
    assert _own_group(lib, L, n=-1) == 1
    assert _own_group(lib, L, n=0) == 0                        # nothing to do: no launch


def test_prefill_dense_workspace_size_and_argument_checks(lib):
    L = _layout()
    # 3 tiles x 8 KV heads x 64 keys x 128 channels x (K fp16 hi + K e4m3 lo + V fp16 = 5 bytes)
    assert lib.echokv_prefill_dense_workspace(C.byref(L), 3) == 3 * 8 * 64 * 128 * 5
    assert lib.echokv_prefill_dense_workspace(C.byref(_layout(head_size=96)), 3) < 0
    assert lib.echokv_prefill_dense_workspace(C.byref(L), -1) < 0
    assert _prefill_dense(lib, _layout(head_size=96)) == 2   # D must be 64 or 128
    assert _prefill_dense(lib, L, hq=30) == 2                 # heads not a multiple of KV heads
    assert _prefill_dense(lib, L, tile_m=32) == 2             # GQA 4 tiles hold 64 tokens
    assert _prefill_dense(lib, L, ws_bytes=1000) != 0         # workspace too small
    assert _prefill_dense(lib, L, n_packs=-1) != 0
    assert _prefill_dense(lib, L, n_q=0) == 0                 # nothing to do: no launch


def test_python_guards_refuse_before_any_device_work():
    """finalize_k refuses a fin table whose rows are not packed at 3 + k_group int64
    (the kernel's stride)."""
    from types import SimpleNamespace

    import torch

    from echokv_amd.kernels.write import finalize_k
    from echokv_amd.write_plan import WriteMeta

    store = SimpleNamespace(layout=TieredLayout(8, 128, 16, 8, 16, 32))
    wide = torch.zeros(2, 40, dtype=torch.long)
    meta = WriteMeta(tok=torch.zeros(4, 1, dtype=torch.long), fin=wide[:, :19], fin_count=torch.ones(1, dtype=torch.long),
                     n_rows=1, n_fin=1)
    with pytest.raises(ValueError, match="row stride 19"):
        finalize_k(store, torch.zeros(1, 8, 128), meta)


@pytest.mark.parametrize("h,d,bs,mem,kg,vg", [(8, 128, 16, 8, 16, 32), (8, 128, 16, 4, 16, 32), (2, 64, 32, 8, 32, 32),
                                              (4, 96, 16, 2, 16, 32), (1, 256, 64, 6, 16, 64)])
def test_aligned_pages_put_every_data_field_on_a_128_byte_line(h, d, bs, mem, kg, vg):
    L = TieredLayout(h, d, bs, mem, kg, vg)
    n = 5
    pages = L.alloc_pages(n, "cpu")
    assert L.aligned_stride % 128 == 0 and pages.stride() == (L.aligned_stride, 1)
    assert pages.shape == (n, L.aligned_stride - L.line_shift) and pages.shape[1] >= L.page_bytes
    assert L.aligned_stride - L.page_bytes < L.line_shift + 128
    o = L.offsets["data"]
    assert all((pages[i].data_ptr() + o) % 128 == 0 for i in range(n))
    end = pages.storage_offset() + (n - 1) * L.aligned_stride + pages.shape[1]
    assert end <= pages.untyped_storage().nbytes()
