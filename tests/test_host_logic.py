"""Host-side logic of the engine that runs without a GPU.

* ``Sequential`` places every state tensor of every layer, nested ones included (a
  residual block's branches, an attention layer's projections, BatchNorm running
  statistics, the positional-encoding table), on its device (network.py:40-90).
* The record of which convolutions have their bias deltas formed by a pending BatchNorm
  pass belongs to the deferral context: it is taken once, and nothing of it survives the
  context, also when the context is left by an exception.
"""

from __future__ import annotations

import pytest
import torch


def _state_tensors(layer):
    from triton_tagi_amd.network import _PLACED_STATE, _all_layers

    out = []
    for sub in _all_layers([layer]):
        if sub.sublayers():
            continue
        for name in _PLACED_STATE:
            t = getattr(sub, name, None)
            if isinstance(t, torch.Tensor):
                out.append((f"{type(sub).__name__}.{name}", t))
    return out


def test_sequential_places_every_nested_state_tensor():
    from triton_tagi_amd import workloads
    from triton_tagi_amd.layers import BatchNorm2D, Conv2D, MultiheadAttentionV2, PositionalEncoding, ResBlock
    from triton_tagi_amd.network import Sequential, _all_layers

    for name in ("resnet18", "transformer"):
        layers = (workloads.resnet18_layers() if name == "resnet18" else workloads.transformer_layers())
        before = [tag for lay in layers for tag, _ in _state_tensors(lay)]
        net = Sequential(layers, device="meta")
        got = [(tag, t) for lay in net.layers for tag, t in _state_tensors(lay)]
        assert len(got) == len(before)
        off = [tag for tag, t in got if t.device.type != "meta"]
        assert not off, f"{name}: not placed: {off}"
        kinds = {type(s).__name__ for s in _all_layers(net.layers)}
        if name == "resnet18":
            assert {"Conv2D", "BatchNorm2D", "ResBlock", "Linear"} <= kinds
            blocks = [lay for lay in net.layers if isinstance(lay, ResBlock)]
            assert any(b.use_projection for b in blocks)
            for b in blocks:
                assert b.device == torch.device("meta")
                for sub in b.sublayers():
                    if isinstance(sub, (Conv2D, BatchNorm2D)):
                        assert sub.mw.device.type == "meta" and sub.device == torch.device("meta")
                    if isinstance(sub, BatchNorm2D):
                        assert sub.running_mean.device.type == "meta" and sub.running_var.device.type == "meta"
        else:
            att = [lay for lay in net.layers if isinstance(lay, MultiheadAttentionV2)][0]
            for p in att.sublayers():
                assert p.mw.device.type == "meta" and p.Sw.device.type == "meta"
            pe = [lay for lay in net.layers if isinstance(lay, PositionalEncoding)][0]
            assert pe.pe_cache.device.type == "meta"


def test_bias_delta_record_is_owned_by_the_deferral_context():
    from triton_tagi_amd.layers import _bn_pending as P

    class Conv:
        pass

    a, b = Conv(), Conv()
    assert P.active() is None and not P.bias_deltas_formed(a)
    with P.defer_bn_parameter_deltas() as ctx:
        ctx._bias_convs.add(id(a))  # what ``add(..., conv=a)`` records
        assert P.active() is ctx
        assert not P.bias_deltas_formed(b)
        assert P.bias_deltas_formed(a)
        assert not P.bias_deltas_formed(a), "the record is taken once"
    with pytest.raises(RuntimeError):
        with P.defer_bn_parameter_deltas() as ctx:
            ctx._bias_convs.add(id(a))
            raise RuntimeError("a step that fails between the BatchNorm pass and the conv's backward")
    assert P.active() is None
    assert not P.bias_deltas_formed(a), "a record survived the failed step"
    with P.defer_bn_parameter_deltas():
        assert not P.bias_deltas_formed(a), "a record from a failed step reached the next one"
