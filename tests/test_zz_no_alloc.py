"""hg_root_tactical_probe_noalloc (no device allocation; per-GPU static
scratch) against hg_root_tactical_probe (caller workspace), both through the
C-ABI, on the same inputs: two calls in a row, the second smaller, and the
size limit rejected without a launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _probe_inputs(ext, B, seed):
    from hive_neuralnet_amd import hive_gpu
    states, _ = hive_gpu.random_positions(B, 7, 150, seed)
    legal, nl = ext.generate_legal_moves_batch(states, B)
    pr = torch.from_numpy((np.random.default_rng(seed).integers(0, 8, size=(B, 256)) / 8.0).astype(np.float32)).cuda()
    return states, legal, nl, pr


def _outs(B):
    return (torch.full((B,), -7, dtype=torch.int64, device="cuda"),
            torch.full((B, 256), 7, dtype=torch.uint8, device="cuda"),
            torch.full((B,), 7, dtype=torch.uint8, device="cuda"))


def _call(lib, name, states, legal, nl, pr, B, flags, outs, ws=None):
    s = torch.cuda.current_stream().cuda_stream
    args = [states.data_ptr(), legal.data_ptr(), nl.data_ptr(), pr.data_ptr(), ctypes.c_int64(B), *flags,
            *[o.data_ptr() for o in outs]]
    if ws is not None:
        args.append(ws.data_ptr())
    return getattr(lib, name)(*args, ctypes.c_void_p(s))


@pytest.mark.parametrize("flags", [(1, 1, 1), (1, 0, 1)], ids=["all-stages", "no-screen"])
def test_noalloc_probe_matches_workspace_probe(flags):
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    lib = ext._lib
    for B, seed in ((4096, 0x51), (1000, 0x52)):  # the second call is smaller: no stale job lists
        states, legal, nl, pr = _probe_inputs(ext, B, seed + flags[1])
        want = _outs(B)
        ws = torch.empty((int(lib.hg_root_tactical_probe_workspace(B)),), dtype=torch.int32, device="cuda")
        assert _call(lib, "hg_root_tactical_probe", states, legal, nl, pr, B, flags, want, ws) == 0
        got = _outs(B)
        assert _call(lib, "hg_root_tactical_probe_noalloc", states, legal, nl, pr, B, flags, got) == 0
        torch.cuda.synchronize()
        for w, g in zip(want, got):
            assert torch.equal(w, g)
        assert int((got[0] >= 0).sum()) > 0  # the cases reach the win stages


def test_noalloc_probe_size_limit():
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    lib = ext._lib
    B = hive_gpu.PROBE_NOALLOC_MAX_ROOTS + 1
    st = torch.zeros((1, 3424), dtype=torch.uint8, device="cuda")
    z = torch.zeros((1,), dtype=torch.int64, device="cuda")
    # rejected before anything is launched (the pointers are never read)
    err = lib.hg_root_tactical_probe_noalloc(st.data_ptr(), st.data_ptr(), st.data_ptr(), st.data_ptr(),
                                             ctypes.c_int64(B), 1, 1, 1, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert err != 0
    with pytest.raises(ValueError, match="at most"):
        ext.root_tactical_probe_batch_noalloc(st, st, st, st, B)
    # the Python binding on a small batch equals the reference-API call
    states, legal, nl, pr = _probe_inputs(ext, 64, 0x53)
    for a, b in zip(ext.root_tactical_probe_batch(states, legal, nl, pr, 64),
                    ext.root_tactical_probe_batch_noalloc(states, legal, nl, pr, 64)):
        assert torch.equal(a, b)


def test_noalloc_binding_orders_calls_across_streams():
    """Two binding calls on two streams, enqueued back to back: the second
    waits for the first (they share the scratch), so both equal the
    workspace probe; hg_probe_scratch_init (the address looked up again, as
    after a device reset) leaves later calls correct."""
    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
    assert ext._lib.hg_probe_scratch_init() == 0
    a = _probe_inputs(ext, 4096, 0x61)
    b = _probe_inputs(ext, 2048, 0x62)
    want_a = ext.root_tactical_probe_batch(*a, 4096)
    want_b = ext.root_tactical_probe_batch(*b, 2048)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        got_a = ext.root_tactical_probe_batch_noalloc(*a, 4096)
    with torch.cuda.stream(s2):
        got_b = ext.root_tactical_probe_batch_noalloc(*b, 2048)
    torch.cuda.synchronize()
    for w, g in zip(want_a + want_b, got_a + got_b):
        assert torch.equal(w, g)
