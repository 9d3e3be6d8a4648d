"""C-ABI checks that need no GPU: libesda.so loads, exports every function
include/*.h declares, and rejects bad descriptions before touching the device."""
import ctypes
import os
import re

import pytest

from apertura_amd import _lib
from apertura_amd.decode import DecodeStep, workspace_bytes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in os.listdir(os.path.join(ROOT, "include")):
        if h.endswith(".h"):
            txt = open(os.path.join(ROOT, "include", h)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(esda_\w+)\s*\(", txt, re.M))
    return sorted(names)


def test_header_declares_and_library_exports_every_symbol():
    names = _declared()
    assert "esda_decode" in names and "esda_decode_raw" in names and "esda_cache_update" in names
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), f"libesda.so does not export {n}"
    assert set(names) == set(_lib.EXPORTS)
    assert L.esda_version() >= 100


def _ws(**kw):
    base = dict(batch=1, num_q_heads=32, num_kv_heads=4, head_dim=512, cap=8448, kv_shared=True,
                scale=512 ** -0.5)
    base.update(kw)
    return workspace_bytes(DecodeStep(**base))


def test_workspace_size_of_the_global_config():
    n = _ws()
    assert n > 256
    # partial count grows with splits: explicit small splits need more workspace
    assert _ws(split_rows=64) > _ws(split_rows=1024)


def _plan_bytes(B, D, slots, heads):
    """Workspace of a plan with `slots` split partials of `heads` query heads each: 256-byte
    status area, the batch prefix table, the (m, l) pairs, then the fp32 partial rows."""
    up = lambda n: (n + 255) // 256 * 256
    parts = slots * heads
    return 256 + up((B + 1) * 8) + up(parts * 8) + parts * D * 4


# The automatic plan of each BASELINE config, pinned through its workspace size:
#   C1  D=256, two workgroups per CU: 8 pairs x 32 splits of the 32-row minimum
#   C2  D=512 shared, one per CU: 4 pairs x 57 splits of 144 rows (whole 16-row tiles)
#   C3  D=256 rings: 128 pairs x 4 splits of 256 rows (512 workgroups)
#   C4  D=512 shared: 4 pairs x 64 splits of 2048 rows
#   C5 local  D=256 rings at B=32: 512 pairs, one split each (the size cannot show kv-head
#             packing: pk heads per slot over 1/pk the slots)
#   C5 global D=512 shared, ragged B=32: 256 balanced shares (one per CU) + one slot per pair
PLANS = [
    ("C1", dict(batch=1, num_q_heads=16, num_kv_heads=8, head_dim=256, cap=1024, window=1024), 8 * 32, 2),
    ("C2", dict(batch=1, num_q_heads=32, num_kv_heads=4, head_dim=512, cap=8193, kv_shared=True), 4 * 57, 8),
    ("C3", dict(batch=8, num_q_heads=32, num_kv_heads=16, head_dim=256, cap=1024, window=1024, ring=True),
     8 * 16 * 4, 2),
    ("C4", dict(batch=1, num_q_heads=32, num_kv_heads=4, head_dim=512, cap=131072, kv_shared=True), 4 * 64, 8),
    ("C5-local", dict(batch=32, num_q_heads=32, num_kv_heads=16, head_dim=256, cap=1024, window=1024, ring=True),
     32 * 16, 2),
    ("C5-global", dict(batch=32, num_q_heads=32, num_kv_heads=4, head_dim=512, cap=32768, kv_shared=True),
     32 * 4 + 256, 8),
]


@pytest.mark.parametrize("name,desc,slots,heads", PLANS, ids=[p[0] for p in PLANS])
def test_automatic_plans_of_the_baseline_configs(name, desc, slots, heads):
    n = workspace_bytes(DecodeStep(scale=1.0, **desc))
    assert n == _plan_bytes(desc["batch"], desc["head_dim"], slots, heads), name


@pytest.mark.parametrize("bad", [
    dict(head_dim=96), dict(head_dim=64), dict(num_q_heads=30), dict(num_q_heads=68),
    dict(cap=0), dict(window=-1), dict(ring=True, window=0), dict(ring=True, window=9000),
    dict(head_stride=100), dict(seq_stride=8), dict(split_rows=40), dict(batch=0),
])
def test_invalid_descriptions_are_rejected(bad):
    with pytest.raises(_lib.EsdaError) as ei:
        _ws(**bad)
    assert ei.value.code == 1
    assert _lib.lib().esda_last_error().decode()


def test_decode_rejects_null_arguments_without_device():
    d = DecodeStep(batch=1, num_q_heads=8, num_kv_heads=1, head_dim=128, cap=64).desc()
    a = _lib.DecodeArgs()
    rc = _lib.lib().esda_decode(ctypes.byref(d), ctypes.byref(a), None)
    assert rc == 1 and b"null" in _lib.lib().esda_last_error()


def test_decode_rejects_small_workspace_without_device():
    d = DecodeStep(batch=1, num_q_heads=8, num_kv_heads=1, head_dim=128, cap=64).desc()
    fake = 0x10000  # never dereferenced: validation fails first
    a = _lib.DecodeArgs(fake, fake, fake, fake, fake + 0x100000, fake, None, fake, fake, 16)
    rc = _lib.lib().esda_decode(ctypes.byref(d), ctypes.byref(a), None)
    assert rc == 4


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_LIB_PATH", str(tmp_path / "libesda.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.lib()


# ------------------------------------------------ ES* layer handle (no device calls)

def test_es_cache_handle_host_side_behaviour(tmp_path):
    """Construction, step counting, the not-implemented members' failure values and
    argument validation run on the host only."""
    from apertura_amd.cache import ESKVCache
    c = ESKVCache(4)
    assert c.seq_len() == 0
    c.mark_step(3)
    assert c.seq_len() == 3
    c.reset()
    assert c.seq_len() == 0
    assert c.save_snapshot(str(tmp_path / "s"), "fp", 1) is False
    assert c.restore_snapshot(str(tmp_path / "s"), "fp") == -1
    assert c.mark_rewind_point(1) is False and c.rewind_to_mark() == -1
    assert c.slot(2) == {"len": 0, "start": 0, "capacity": 0, "lost": False, "shared": False, "raw": False,
                         "q8": False}
    with pytest.raises(_lib.EsdaError) as ei:
        c.slot(4)
    assert ei.value.code == 1
    view = _lib.View()
    rc = _lib.lib().esda_cache_update(c._h, 0, None, None, 2, 1, 128, 0, 1, None, ctypes.byref(view),
                                      ctypes.byref(view))
    assert rc == 1 and b"null" in _lib.lib().esda_last_error()
    rc = _lib.lib().esda_cache_current(c._h, 1, 1, ctypes.byref(view), ctypes.byref(view))
    assert rc == 2  # no rows yet: std::runtime_error
    q8v = _lib.Q8View()
    assert _lib.lib().esda_cache_current_raw_q8(c._h, 1, ctypes.byref(q8v)) == 2  # no q8 rows
    rc = _lib.lib().esda_cache_update_raw_q8(c._h, 0, None, 2, 1, None, ctypes.byref(q8v))
    assert rc == 1 and b"null" in _lib.lib().esda_last_error()
    rc = _lib.lib().esda_cache_decode_raw_q8(c._h, 0, None, 16, None, 2, None, 1e-6, None, 0, None, None)
    assert rc == 1
    rc = _lib.lib().esda_decode_attn_global_q8(None, 16, None, None, None, 2, 1, 1, None, 1e-6, None, 0, None, None)
    assert rc == 1
    with pytest.raises(_lib.EsdaError):
        ESKVCache(0)


def test_raw_descriptions_are_validated_without_device():
    from apertura_amd.decode import RawStep, raw_workspace_bytes
    assert raw_workspace_bytes(RawStep(batch=1, num_q_heads=32, num_kv_heads=4, cap=131072)) > 256
    for bad in (dict(head_dim=256), dict(num_q_heads=31), dict(cap=0), dict(eps=-1.0),
                dict(split_rows=40)):
        kw = dict(batch=1, num_q_heads=32, num_kv_heads=4, cap=1024)
        kw.update(bad)
        with pytest.raises(_lib.EsdaError) as ei:
            raw_workspace_bytes(RawStep(**kw))
        assert ei.value.code == 1


def test_rope_table_arguments_are_validated_without_device():
    import ctypes
    L = _lib.lib()
    buf = (ctypes.c_uint8 * 512)()
    addr = (ctypes.addressof(buf) + 15) // 16 * 16
    assert L.esda_rope_table(None, 4, addr, None) == 1          # null inv_freq
    assert L.esda_rope_table(addr, 4, None, None) == 1          # null table
    assert L.esda_rope_table(addr, -1, addr, None) == 1         # negative rows
    assert L.esda_rope_table(addr, 4, addr + 4, None) == 1      # table not 16-byte aligned


def test_prefill_descriptions_are_validated_without_device():
    """esda_prefill's plan is host-side: malformed descriptions fail with
    ESDA_ERR_INVALID_ARGUMENT before any device call; splits size the workspace."""
    from apertura_amd._lib import EsdaError
    from apertura_amd.prefill import PrefillStep, prefill_workspace_bytes
    good = dict(num_q_heads=32, num_kv_heads=4, head_dim=512, seq_q=512, seq_k=16384, q_pos0=15872, k_pos0=0)
    n = prefill_workspace_bytes(PrefillStep(**good))
    assert n > 0  # 16 query tiles per kv head: the keys are split to cover the CUs
    assert prefill_workspace_bytes(PrefillStep(**{**good, "seq_q": 16384, "q_pos0": 0})) == 0  # enough tiles
    # a 512-query sliding chunk at GQA 32/16: 128 tiles of 128 rows would split the keys; the
    # 64-row tiles of the stage-halves kernel cover the 256 CUs, so no partials
    local = dict(num_q_heads=32, num_kv_heads=16, head_dim=256, seq_q=512, seq_k=1536, q_pos0=15872,
                 k_pos0=14848, window=1024)
    assert prefill_workspace_bytes(PrefillStep(**local)) == 0
    assert prefill_workspace_bytes(PrefillStep(**{**local, "num_kv_heads": 4, "num_q_heads": 8})) > 0
    for bad in (dict(head_dim=64), dict(num_q_heads=30), dict(seq_q=0), dict(window=-1),
                dict(k_pos0=15873),                              # the first query's own key missing
                dict(seq_k=100),                                 # the last queries' keys missing
                dict(split_keys=48), dict(scale=0.0), dict(q_head_stride=12),
                dict(q_pos0=2 ** 31 - 100)):
        with pytest.raises(EsdaError) as ei:
            prefill_workspace_bytes(PrefillStep(**{**good, **bad}))
        assert ei.value.code == 1, bad
