"""spk_lm_head_argmax_noalloc (static device scratch, no workspace argument)
against spk_lm_head_argmax (caller workspace) through the C ABI: two calls in
a row, the second with a smaller vocabulary, then the first size again; the
fp16 logits and the argmax index must be identical bit for bit.  Sizes beyond
the static scratch are rejected before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_VOCAB = 262144  # SPK_LM_HEAD_NOALLOC_MAX_VOCAB


def _run_both(lib, W, x, vocab, hidden, dev):
    s = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.spk_lm_head_workspace_size(vocab)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    ref_logits = torch.empty(vocab, dtype=torch.float16, device=dev)
    ref_idx = torch.full((1,), -1, dtype=torch.int32, device=dev)
    rc = lib.spk_lm_head_argmax(W.data_ptr(), x.data_ptr(), vocab, hidden, ref_logits.data_ptr(),
                                ref_idx.data_ptr(), ws.data_ptr(), ws_bytes, s)
    assert rc == 0, lib.spk_last_error()
    logits = torch.empty(vocab, dtype=torch.float16, device=dev)
    idx = torch.full((1,), -1, dtype=torch.int32, device=dev)
    rc = lib.spk_lm_head_argmax_noalloc(W.data_ptr(), x.data_ptr(), vocab, hidden, logits.data_ptr(),
                                        idx.data_ptr(), s)
    assert rc == 0, lib.spk_last_error()
    idx_only = torch.full((1,), -1, dtype=torch.int32, device=dev)
    rc = lib.spk_lm_head_argmax_noalloc(W.data_ptr(), x.data_ptr(), vocab, hidden, None,
                                        idx_only.data_ptr(), s)
    assert rc == 0, lib.spk_last_error()
    torch.cuda.synchronize()
    return (ref_logits.cpu().numpy().view(np.uint16), int(ref_idx.cpu()[0]),
            logits.cpu().numpy().view(np.uint16), int(idx.cpu()[0]), int(idx_only.cpu()[0]))


def test_noalloc_lm_head_matches_workspace_entry_point(dev, oracle):
    from spock_amd import _lib, synth
    lib = _lib.lib()
    hidden = 1024
    big, small = 248320, 50021
    f16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(dev)
    W = f16(synth.gemv_weights(big, hidden, seed=61))
    x = f16(synth.gemv_input(hidden, seed=62))
    x2 = f16(synth.gemv_input(hidden, seed=63))
    print("[noalloc lm_head] vocab 248320, then 50021, then 248320", flush=True)
    for vocab, xv in ((big, x), (small, x2), (big, x2)):
        rl, ri, gl, gi, gi2 = _run_both(lib, W, xv, vocab, hidden, dev)
        assert np.array_equal(gl, rl)
        assert gi == ri == gi2
        assert 0 <= gi < vocab
    # the small call against the CPU oracle as well
    e_idx, e_logits = oracle.lm_head_argmax(W[:small].cpu().numpy().view(np.uint16),
                                            x2.cpu().numpy().view(np.uint16))
    _, ri, gl, gi, _ = _run_both(lib, W, x2, small, hidden, dev)
    assert gi == e_idx and np.array_equal(gl, e_logits)


def test_noalloc_lm_head_rejects_sizes_beyond_scratch(dev):
    from spock_amd import _lib
    lib = _lib.lib()
    s = torch.cuda.current_stream().cuda_stream
    W = torch.empty(16, 1024, dtype=torch.float16, device=dev)  # never read: rejected first
    x = torch.zeros(1024, dtype=torch.float16, device=dev)
    idx = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = lib.spk_lm_head_argmax_noalloc(W.data_ptr(), x.data_ptr(), MAX_VOCAB + 1, 1024, None,
                                        idx.data_ptr(), s)
    assert rc == -2 and b"static scratch limit" in lib.spk_last_error()
    rc = lib.spk_lm_head_argmax_noalloc(W.data_ptr(), x.data_ptr(), 16, 1000, None, idx.data_ptr(), s)
    assert rc == -2
    rc = lib.spk_lm_head_argmax_noalloc(None, x.data_ptr(), 16, 1024, None, idx.data_ptr(), s)
    assert rc == -1
