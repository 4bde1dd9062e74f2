"""vasc_select_blocks_noalloc: the selection entry point that allocates
nothing, checked through the C-ABI against vasc_select_blocks (caller
workspace) on the same inputs, bit for bit, on two calls in a row (the
second smaller, so stale scratch contents from the first call are present).
"""
import ctypes

import pytest
import torch

from vasc_amd import _lib, ops


def _ptr(t):
    return None if t is None else t.data_ptr()


def _inputs(B, H, Q, K, seed, dev):
    g = torch.Generator().manual_seed(seed)
    P = (K + 1) // 2
    score = torch.softmax(torch.randn(B, H, Q, K, generator=g) * 3.0, dim=-1)
    inn = torch.rand(B, H, P, generator=g) * 0.5
    inn[..., ::7] = 0.0  # zero-innovation pairs
    debt = torch.rand(B, H, P, generator=g) * 0.01
    pend = torch.rand(B, H, P, generator=g) * 0.01
    prev = torch.rand(B, H, P, generator=g) * 0.01
    return [t.float().contiguous().to(dev) for t in (score, inn, debt, pend, prev)]


def _run(entry, B, H, Q, K, tensors, mode, topk, force_last, sink, ws=None):
    score, inn, debt, pend, prev = tensors
    dev = score.device
    P = (K + 1) // 2
    vasc = mode == _lib.MODE_VASC
    maxc = min(topk + int(force_last), K) if not vasc else min(topk, K)
    width = maxc + sink
    out = {
        "index": torch.full((B, H, Q, width), -7, device=dev, dtype=torch.int32),
        "count": torch.full((B, H, Q), -7, device=dev, dtype=torch.int32),
        "priority": torch.full((B, H, Q, K), -7.0, device=dev, dtype=torch.float32),
    }
    if vasc:
        for name in ("debt", "arrival", "service"):
            out[name] = torch.full((B, H, P), -7.0, device=dev, dtype=torch.float32)
        out["gate"] = torch.full((1,), -7, device=dev, dtype=torch.int32)
    args = [score.data_ptr(), _ptr(inn if vasc else None), B, H, Q, K, int(mode), int(topk), None, None,
            int(force_last), int(maxc if vasc else 0), int(sink),
            _ptr(debt if vasc else None), _ptr(pend if vasc else None), _ptr(prev if vasc else None),
            _ptr(out.get("debt")), _ptr(out.get("arrival")), _ptr(out.get("service")), _ptr(out.get("gate")),
            out["priority"].data_ptr() if vasc else None, None, out["index"].data_ptr(), width,
            out["count"].data_ptr()]
    if entry == "vasc_select_blocks":
        args += [_ptr(ws), 0 if ws is None else ws.numel()]
    args.append(ops._stream())
    _lib.call(entry, *args)
    return out


def _equal(a, b):
    assert a.keys() == b.keys()
    for k in a:
        if a[k].dtype == torch.float32:
            assert torch.equal(a[k].view(torch.int32), b[k].view(torch.int32)), k
        else:
            assert torch.equal(a[k], b[k]), k


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [_lib.MODE_VASC, _lib.MODE_TOPK])
def test_noalloc_matches_workspace_entry_point(mode):
    dev = torch.device("cuda:0")
    # first call at C2's per-layer shape, then a smaller one with an odd key
    # count, a forced tail and different sink width
    for (B, H, Q, K, topk, fl, sink, seed) in ((1, 16, 259, 518, 129, 0, 3, 1), (2, 3, 37, 131, 20, 1, 1, 2)):
        print(f"[no-alloc] mode {mode} B={B} H={H} Q={Q} K={K}", flush=True)
        t = _inputs(B, H, Q, K, seed, dev)
        ws = ops.select_workspace(B, H, Q, K, dev) if mode == _lib.MODE_VASC else None
        ref = _run("vasc_select_blocks", B, H, Q, K, t, mode, topk, fl, sink, ws)
        got = _run("vasc_select_blocks_noalloc", B, H, Q, K, t, mode, topk, fl, sink)
        torch.cuda.synchronize()
        _equal(got, ref)
        cnt = got["count"].cpu().numpy()
        assert (cnt >= 1).all() and (cnt <= topk + fl + sink).all()
    # a third call at the first shape again gives the same bits as the first
    B, H, Q, K = 1, 16, 259, 518
    t = _inputs(B, H, Q, K, 1, dev)
    ws = ops.select_workspace(B, H, Q, K, dev) if mode == _lib.MODE_VASC else None
    _equal(_run("vasc_select_blocks_noalloc", B, H, Q, K, t, mode, 129, 0, 3),
           _run("vasc_select_blocks", B, H, Q, K, t, mode, 129, 0, 3, ws))


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """Checked before any HIP call (no GPU needed): a workspace above
    VASC_SELECT_SCRATCH_BYTES is refused with a clear error."""
    lib = _lib.load()
    limit = 32 << 20
    B, H, Q, K = 1, 16, 4096, 8192
    assert lib.vasc_select_workspace_size(B, H, Q, K) > limit
    assert lib.vasc_select_workspace_size(1, 16, 2048, 4096) <= limit
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced
    rc = lib.vasc_select_blocks_noalloc(fake, fake, B, H, Q, K, _lib.MODE_VASC, 100, None, None, 0, 100, 0,
                                        None, None, None, fake, fake, fake, None, None, None, fake, 100, fake, None)
    assert rc == 1
    msg = lib.vasc_last_error()
    assert b"scratch" in msg and b"maximum" in msg
