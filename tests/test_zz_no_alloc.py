"""GPU: the allocation-free decode layer (oc_decode_layer_noalloc).

Called through the C ABI with the argument struct a DecodeLayer builds for
oc_decode_layer, but with fresh outputs, and compared with oc_decode_layer's
outputs bit for bit (the same kernels on the same data): attention output,
scores, permutation and count.  Two calls in a row, the second on a smaller
layer, so the second runs in scratch memory that still holds the first
call's contents.
"""

import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev, seq, evict, seed):
    from orthocache_amd import _ops, workloads

    wl = workloads.c2(dev, seed=seed, seq=seq)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, evict)
    return wl, _ops.DecodeLayer(wl.q, wl.k, wl.v, tau, zmax)


def _noalloc(layer):
    """oc_decode_layer_noalloc on the layer's inputs and thresholds, writing
    fresh output tensors; returns them."""
    from orthocache_amd import _native as N

    outs = {"out": torch.empty_like(layer.out), "tau_max": torch.empty_like(layer.tau_max),
            "zeta": torch.empty_like(layer.zeta), "indices": torch.empty_like(layer.indices),
            "num_active": torch.empty_like(layer.num_active)}
    for t in outs.values():
        t.fill_(-7)  # anything the call does not write shows up
    a = N.LayerArgs.from_buffer_copy(layer.args)
    a.out = outs["out"].data_ptr()
    a.tau_max = outs["tau_max"].data_ptr()
    a.zeta = outs["zeta"].data_ptr()
    a.indices = outs["indices"].data_ptr()
    a.num_active = outs["num_active"].data_ptr()
    L = N.lib()
    rc = L.oc_decode_layer_noalloc(C.byref(a), N.stream_ptr(layer.device))
    assert rc == 0, L.oc_last_error()
    return outs


def test_noalloc_layer_matches_decode_layer(dev):
    from orthocache_amd import _native as N

    ref = {}
    got = {}
    # 64K tokens (10 MiB of scratch), then 16K tokens with other data
    for name, seq, evict, seed in (("large", 65536, 0.9, 2), ("small", 16384, 0.75, 5)):
        wl, layer = _layer(dev, seq, evict, seed)
        need = int(N.lib().oc_decode_layer_workspace_size(C.byref(layer.args)))
        assert 0 < need <= N.NOALLOC_SCRATCH_BYTES
        print(f"noalloc: {name} layer, {seq} tokens, workspace {need} bytes", flush=True)
        layer.run()
        ref[name] = {"out": layer.out.clone(), "tau_max": layer.tau_max.clone(), "zeta": layer.zeta.clone(),
                     "indices": layer.indices.clone(), "num_active": layer.num_active.clone()}
        got[name] = _noalloc(layer)
        torch.cuda.synchronize()
        for key, r in ref[name].items():
            assert torch.equal(got[name][key], r), (name, key)
        nb = seq // 512
        assert int(got[name]["num_active"][0]) == int(round(nb * (1 - evict)))
    # a repeat of the large layer after the small one
    wl, layer = _layer(dev, 65536, 0.9, 2)
    again = _noalloc(layer)
    torch.cuda.synchronize()
    for key, r in ref["large"].items():
        assert torch.equal(again[key], r), ("repeat", key)
