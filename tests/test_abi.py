"""C-ABI checks that need no GPU: libesda.so loads, exports every function
include/esda.h declares, and rejects bad descriptions before touching the device."""
import ctypes
import os
import re

import pytest

from apertura_amd import _lib
from apertura_amd.decode import DecodeStep, workspace_bytes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    txt = open(os.path.join(ROOT, "include", "esda.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(esda_\w+)\s*\(", txt, re.M)))


def test_header_declares_and_library_exports_every_symbol():
    names = _declared()
    assert "esda_decode" in names and len(names) >= 7
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
