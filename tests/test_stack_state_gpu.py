"""Snapshot / crop and saved states of the mixer stack (Lm::snapshot / crop / save_state /
load_state; engine hybrid.rs:1029-1070, next.rs:2442-2578). The stack's kernels are
deterministic, so re-feeding the same tokens after a crop, or continuing from a loaded state,
must reproduce the original outputs bit for bit."""
import pytest
import torch

from aegist_mixer import ops
from aegist_mixer import state_file

from test_stack_gpu import CFG, KINDS, make_layers

pytestmark = pytest.mark.gpu


def _stack(dev, B=1, cap=128, seed=0):
    _, dl = make_layers(seed, dev)
    return ops.HybridStack(CFG, KINDS, dl, max_batch=B, max_tokens=B * 64, max_context=cap), dl


def _feed(stack, xs):
    outs = []
    for x in xs:
        y = x.clone()
        stack.forward(y)
        outs.append(y)
    torch.cuda.synchronize()
    return outs


def _inputs(dev, B, sizes, seed):
    g_ = torch.Generator().manual_seed(seed)
    return [torch.randn(B, t, CFG["d_model"], generator=g_).to(dev) for t in sizes]


def test_crop_to_snapshot_then_refeed_is_identical(dev):
    B = 2
    stack, _keep = _stack(dev, B=B)
    pre, tail = _inputs(dev, B, [40], 1), _inputs(dev, B, [20, 1, 1, 1], 2)
    _feed(stack, pre)
    stack.snapshot()
    first = _feed(stack, tail)
    assert stack.length == 63
    assert stack.crop(100) == 63 and stack.crop(63) == 63  # n >= length keeps everything
    assert stack.crop(50) == 40
    again = _feed(stack, tail)
    for a, b in zip(first, again):
        assert torch.equal(a, b)
    stack.close()


def test_snapshot_slot_policy(dev):
    stack, _keep = _stack(dev)
    xs = _inputs(dev, 1, [8, 8, 8], 3)
    for x in xs:
        _feed(stack, [x])
        stack.snapshot()
        stack.snapshot()  # a second snapshot at the same length takes no slot
    # two slots: the snapshot at 8 was replaced by the one at 24
    assert stack.crop(12) == 0 and stack.length == 0
    for x in xs:
        _feed(stack, [x])
        if stack.length < 24:
            stack.snapshot()
    assert stack.crop(20) == 16
    assert stack.crop(10) == 8
    assert stack.crop(3) == 0
    stack.close()


def test_crop_without_snapshot_resets_state(dev):
    stack, _keep = _stack(dev)
    xs = _inputs(dev, 1, [16, 16], 4)
    fresh = _feed(stack, xs[:1])
    _feed(stack, xs[1:])
    assert stack.crop(5) == 0 and stack.length == 0
    assert torch.equal(_feed(stack, xs[:1])[0], fresh[0])
    stack.close()


def test_save_load_round_trip(dev, tmp_path):
    stack, keep = _stack(dev)
    pre, dec = _inputs(dev, 1, [30], 5), _inputs(dev, 1, [1, 1], 6)
    _feed(stack, pre)
    toks = list(range(100, 130))
    path = tmp_path / "s.aegstate"
    stack.save_state(path, toks, key="mixer-test")
    want = _feed(stack, dec)
    # payload size: K and V rows of every attention layer, conv + recurrent state of every
    # recurrent layer
    C = 2 * CFG["hk"] * 128 + CFG["hv"] * 128
    na, nd = KINDS.count("attn"), KINDS.count("delta")
    nbytes = na * CFG["n_kv"] * 30 * 256 * 2 * 2 + nd * (C * 3 * 4 + CFG["hv"] * 128 * 128 * 4)
    assert stack.state_bytes(30) == nbytes
    raw = path.read_bytes()
    assert raw[:8] == b"AEGSTATE" and len(raw) == 16 + int.from_bytes(raw[8:16], "little") + nbytes
    other, _keep2 = _stack(dev)
    assert other.load_state(path, key="mixer-test") == toks
    assert other.length == 30
    got = _feed(other, dec)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
    # the load took a snapshot at 30
    assert other.crop(31) == 30
    with pytest.raises(state_file.StateFileError, match="another brain"):
        other.load_state(path, key="other")
    assert other.length == 0
    stack.close()
    other.close()
