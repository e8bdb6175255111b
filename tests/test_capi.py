"""The C ABI surface, without a GPU: the library loads, exports every
function include/spock_hip.h declares, and rejects invalid arguments before
touching the device."""
import ctypes as C
import re

import pytest

from conftest import ROOT


def _declared(header="spock_hip.h"):
    hdr = (ROOT / "include" / header).read_text()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    return sorted(set(re.findall(r"\b(spk_[a-z0-9_]+)\s*\(", hdr)))


def test_header_and_binding_agree():
    from spock_amd import _lib
    assert set(_declared()) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from spock_amd import _lib
    lib = _lib.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.spk_abi_version() >> 16 == 1


def test_struct_layouts_match_header():
    from spock_amd import _lib
    # field order and C sizes of the argument structs (x86-64 SysV)
    assert C.sizeof(_lib.SpkMatvecDesc) == 32
    assert _lib.SpkChunkArgs.q.offset == 32 and _lib.SpkChunkArgs.workspace_bytes.offset == 136
    assert _lib.SpkDecodeArgs.qkv.offset == 24 and C.sizeof(_lib.SpkDecodeArgs) == 136


def test_argument_errors_without_device():
    from spock_amd import _lib
    lib = _lib.lib()
    assert lib.spk_chunk_prefill(None, None) == -1                      # SPK_ERR_NULL
    a = _lib.SpkChunkArgs()
    a.num_heads, a.total_tokens, a.key_dim, a.value_dim, a.chunk_size = 16, 10, 64, 128, 64
    assert lib.spk_chunk_prefill(C.byref(a), None) == -2                # unsupported key_dim
    assert b"key_dim" in lib.spk_last_error()
    a.key_dim = 128
    a.num_seqs = 1
    assert lib.spk_chunk_prefill(C.byref(a), None) == -1                # out_state/workspace missing
    assert lib.spk_matvec_f16(None, None, None, 4, 64, None) == -1
    assert lib.spk_matvec_f16(1, 1, 1, 4, 63, None) == -2               # in_dim % 64
    assert lib.spk_matvec_f16_order(1, 1, 1, 4, 63, 0, None) == -2      # spans: in_dim % 64
    assert lib.spk_matvec_f16_order(1, 1, 1, 4, 64, 3, None) == -5      # unknown order (SPK_ERR_ARG)
    assert b"order" in lib.spk_last_error()
    assert lib.spk_matvec_f16_order(None, 1, 1, 4, 63, 1, None) == -1
    assert lib.spk_matvec_f16_order(1, 1, 1, 4, 0, 2, None) == -2       # in_dim <= 0
    assert lib.spk_matvec_f16_order(1, 1, 1, 0, 63, 1, None) == 0       # nothing to do
    assert lib.spk_argmax_f16(1, 0, 1, None) == -2
    d = _lib.SpkDecodeArgs()
    d.batch, d.num_heads = 1, 16
    assert lib.spk_deltanet_decode_step(C.byref(d), None) == -1         # qkv missing
    assert lib.spk_chunk_prefill_workspace_size(16, 104, 1, 64) == (2 + 1) * 16 * 50176
    assert lib.spk_lm_head_workspace_size(248320) % 256 == 0
    assert lib.spk_deltanet_norm_gate_f16(None, 1, 1, 16, 128, 1e-6, None) == -1   # io missing
    assert lib.spk_deltanet_norm_gate_f16(1, 1, 1, 16, 64, 1e-6, None) == -2      # head_dim != 128
    assert lib.spk_deltanet_norm_gate_f16(1, 1, 1, 0, 128, 1e-6, None) == -2      # no heads
    assert lib.spk_deltanet_inproj_step(None, None, None, None, None) == -1
    gi = _lib.SpkGemvInput()
    gi.kind, gi.in_dim, gi.x, gi.x2 = _lib.SPK_GEMV_IN_PLAIN, 1024, 16, 16
    outs = (_lib.SpkGemvOutput * 3)()
    for o, n, y in zip(outs, (4096, 512, 512), (4096, 8192, 12288)):
        o.W, o.y, o.out_dim = 16, y, n
    aa = _lib.SpkAttnArgs()
    assert lib.spk_attention_inproj(None, outs, C.byref(aa), None) == -1
    assert lib.spk_attention_inproj(C.byref(gi), outs, C.byref(aa), None) == -5   # not the RMSNorm kind
    gi.kind = _lib.SPK_GEMV_IN_RMSNORM
    assert lib.spk_attention_inproj(C.byref(gi), outs, C.byref(aa), None) == -1   # kv_cache/pos_dev missing
    aa.kv_cache, aa.pos_dev, aa.max_seq = 256, 256, 2048
    assert lib.spk_attention_inproj(C.byref(gi), outs, C.byref(aa), None) == -5   # qg/k/v are not the outputs
    aa.qg, aa.k, aa.v = 4096, 8192, 12288
    outs[1].out_dim = 256
    assert lib.spk_attention_inproj(C.byref(gi), outs, C.byref(aa), None) == -2   # k rows != 512


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from spock_amd import _lib
    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(_lib.SpockError, match="no CPU fallback"):
        _lib.lib()


def test_model_header_binding_and_exports():
    """include/spock_model.h (the session surface) against spock_amd/model.py
    and libspock_hip_host.so's exports."""
    from spock_amd import model
    assert set(_declared("spock_model.h")) == set(model.SIGNATURES)
    lib = model.lib()
    for name in _declared("spock_model.h"):
        assert hasattr(lib, name), name
    assert C.sizeof(model.SpkGenerateStats) == 40


def test_model_session_errors_without_device(tmp_path):
    from spock_amd import model
    with pytest.raises(model.ModelError, match="text_repack_manifest.json|cannot open|No such"):
        model.Session(tmp_path / "absent")
    assert model.lib().spk_model_info(None, None, None, None) == -1
    assert model.lib().spk_artifact_write_synthetic(str(tmp_path / "x").encode(), 0, 10, 1) == -1
