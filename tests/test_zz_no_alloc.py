"""rte_pack_index_noalloc (the pack with its scratch in a static device array) against
rte_pack_index with a caller workspace, through the C ABI: bit-identical outputs on two calls
in a row, the second one smaller, and a clear error for sizes beyond the static array."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _zipf_ids(rng, T, C, k):
    p = 1.0 / np.arange(1, C + 1) ** 1.1
    p /= p.sum()
    # k distinct clusters per token, Zipf-skewed (Gumbel top-k sampling without replacement)
    keys = np.log(p)[None, :] + rng.gumbel(size=(T, C))
    ids = np.argsort(-keys, axis=1)[:, :k].astype(np.int32)
    ids[rng.random(ids.shape) < 0.01] = -1  # a few dropped pairs (invalid cluster ids)
    return ids


def _outputs(P, C, dev):
    return dict(off=torch.full((C + 1,), -7, dtype=torch.int32, device=dev),
                tok=torch.full((P,), -7, dtype=torch.int32, device=dev),
                pos=torch.full((P,), -7, dtype=torch.int32, device=dev),
                sop=torch.full((P,), -7, dtype=torch.int32, device=dev),
                wos=torch.full((P,), -7.0, dtype=torch.float32, device=dev),
                inv=torch.zeros((1,), dtype=torch.int32, device=dev))


def _call(lib_call, name, cl, w, P, C, k, o, ws=None):
    from rte_amd import _lib

    args = [cl.data_ptr(), P, C, k, w.data_ptr(), o["off"].data_ptr(), o["tok"].data_ptr(), o["pos"].data_ptr(),
            o["sop"].data_ptr(), o["wos"].data_ptr(), o["inv"].data_ptr()]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    lib_call(name, *args, _lib.stream_ptr())


def test_pack_noalloc_matches_pack_index_twice():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready")
    dev = "cuda"
    rng = np.random.default_rng(5)
    lib = _lib.load()
    for T, C, k in ((16384, 256, 16), (3000, 64, 8)):  # second call smaller: stale scratch must not leak
        P = T * k
        print(f"pack_noalloc case T={T} C={C} k={k}", flush=True)
        ids = _zipf_ids(rng, T, C, k)
        cl = torch.from_numpy(ids).to(dev)
        w = torch.from_numpy(rng.random((T, k), dtype=np.float32)).to(dev)
        ref = _outputs(P, C, dev)
        nb = lib.rte_pack_workspace_bytes(P, C)
        assert nb <= lib.rte_pack_index_noalloc_max_bytes()
        ws = torch.empty((nb,), dtype=torch.uint8, device=dev)
        _call(_lib.call, "rte_pack_index", cl, w, P, C, k, ref, ws)
        got = _outputs(P, C, dev)
        _call(_lib.call, "rte_pack_index_noalloc", cl, w, P, C, k, got)
        torch.cuda.synchronize()
        for key in ref:
            assert torch.equal(ref[key], got[key]), key
        # the pack itself: slots ascend by pair inside each cluster, and every valid pair has one slot
        off = got["off"].cpu().numpy()
        assert off[-1] == int((ids >= 0).sum())
        assert int(got["inv"].item()) == int((ids < 0).sum())


def test_pack_noalloc_rejects_oversize():
    from rte_amd import _lib

    lib = _lib.load()
    P, C = 1 << 22, 4096
    assert lib.rte_pack_workspace_bytes(P, C) > lib.rte_pack_index_noalloc_max_bytes()
    rc = lib.rte_pack_index_noalloc(None, P, C, 1, None, None, None, None, None, None, None, None)
    assert rc != 0
    assert "static" in _lib.last_error()
