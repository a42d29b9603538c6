"""ltkv_set_attention_engine on metadata-only caches (no GPU): the engines it
accepts, per pool dtype, and the errors it returns."""

import pytest

from langtrain_studio_amd import KvCache, KvError, _lib


def test_engine_setter_accepts_and_refuses():
    for dtype in ("f16", "f32"):
        c = KvCache(1, 256, 64, dtype=dtype, device=_lib.NO_DEVICE)
        c.set_attention_engine("valu")
        c.set_attention_engine("auto")
        c.close()
    q8 = KvCache(1, 256, 64, dtype="q8_0", device=_lib.NO_DEVICE)
    q8.set_attention_engine("auto")
    with pytest.raises(KvError) as e:
        q8.set_attention_engine("valu")
    assert e.value.code == _lib.ERR_ARG and "Q8_0" in str(e.value)
    with pytest.raises(ValueError):
        q8.set_attention_engine("mfma")
    q8.close()


def test_engine_setter_rejects_unknown_codes():
    lib = _lib.load()
    c = KvCache(1, 64, 64, device=_lib.NO_DEVICE)
    assert lib.ltkv_set_attention_engine(c._h, 7) == _lib.ERR_ARG
    assert lib.ltkv_set_attention_engine(None, _lib.ENGINE_VALU) == _lib.ERR_ARG
    c.close()
