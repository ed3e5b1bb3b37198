"""The allocation-free routing permutation (moe_permute_fwd_noalloc) against
moe_permute_fwd, through the C ABI: bit-identical outputs on two calls in a
row, the second smaller (its fixed scratch keeps the first call's contents),
replays of a captured HIP graph, no device allocation by a call, and the size
limit refused before any launch."""

import ctypes

import pytest
import torch

from parallel_amd import _lib

DEV = "cuda"
BF = torch.bfloat16


def _outputs(T, k, nb, H, device):
    S = T * k
    i32 = dict(dtype=torch.int32, device=device)
    return (torch.empty(S, H, dtype=BF, device=device), torch.empty(S, **i32), torch.empty(S, **i32),
            torch.empty(nb, **i32), torch.empty(nb, **i32))


def _run(name, hidden, ids, divisor, nb):
    T, k = ids.shape
    H = hidden.shape[1]
    rows, perm, pos, counts, offsets = _outputs(T, k, nb, H, hidden.device)
    lib = _lib.load()
    stream = _lib.stream_of(hidden)
    common = (hidden.data_ptr(), T, H, ids.data_ptr(), k, divisor, nb, rows.data_ptr(), perm.data_ptr(),
              pos.data_ptr(), counts.data_ptr(), offsets.data_ptr())
    if name == "moe_permute_fwd":
        ws = torch.empty(max(lib.moe_permute_workspace_bytes(T * k, nb), 16), dtype=torch.uint8, device=hidden.device)
        _lib.check(lib.moe_permute_fwd(*common, ws.data_ptr(), ws.numel(), stream), name)
    else:
        _lib.check(lib.moe_permute_fwd_noalloc(*common, stream), name)
    return rows, perm, pos, counts, offsets


@pytest.mark.gpu
def test_noalloc_permute_equals_permute_on_consecutive_calls():
    g = torch.Generator().manual_seed(0)
    cases = [(4096, 8, 1, 128, 2048), (300, 4, 16, 5, 64)]  # (T, k, divisor, buckets, H); the second is smaller
    for T, k, divisor, nb, H in cases:
        hidden = torch.randn(T, H, generator=g).to(BF).to(DEV)
        ids = torch.randint(-2, divisor * (nb + 1), (T, k), generator=g).to(DEV)
        want = _run("moe_permute_fwd", hidden, ids, divisor, nb)
        got = _run("moe_permute_fwd_noalloc", hidden, ids, divisor, nb)
        torch.cuda.synchronize()
        for label, a, b in zip(("rows", "perm", "pos_of_slot", "counts", "offsets"), got, want):
            n = int(want[4][-1]) if label == "rows" else None  # sentinel rows are written as zeros by both
            assert torch.equal(a if n is None else a[:n], b if n is None else b[:n]), f"T={T} {label}"
        assert not got[0][int(want[4][-1]):].any()


@pytest.mark.gpu
def test_noalloc_permute_at_its_largest_size():
    """The largest size the scratch takes at 128 buckets: 2032 chunks of 512
    routes (1,048,512 of its 1,048,576 bytes), routing only (no rows)."""
    lib = _lib.load()
    T, k, nb = 130048, 8, 128
    assert lib.moe_permute_workspace_bytes(T * k, nb) == 2032 * 129 * 4
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, nb + 1, (T, k), generator=g).to(DEV)
    S = T * k
    outs = {}
    for name in ("moe_permute_fwd", "moe_permute_fwd_noalloc"):
        i32 = dict(dtype=torch.int32, device=DEV)
        perm, pos, counts, offsets = (torch.empty(S, **i32), torch.empty(S, **i32), torch.empty(nb, **i32),
                                      torch.empty(nb, **i32))
        common = (None, T, 8, ids.data_ptr(), k, 1, nb, None, perm.data_ptr(), pos.data_ptr(), counts.data_ptr(),
                  offsets.data_ptr())
        stream = _lib.stream_of(ids)
        if name == "moe_permute_fwd":
            ws = torch.empty(lib.moe_permute_workspace_bytes(S, nb), dtype=torch.uint8, device=DEV)
            _lib.check(lib.moe_permute_fwd(*common, ws.data_ptr(), ws.numel(), stream), name)
        else:
            _lib.check(lib.moe_permute_fwd_noalloc(*common, stream), name)
        outs[name] = (perm, pos, counts, offsets)
    torch.cuda.synchronize()
    for label, a, b in zip(("perm", "pos_of_slot", "counts", "offsets"), outs["moe_permute_fwd_noalloc"],
                           outs["moe_permute_fwd"]):
        assert torch.equal(a, b), label


@pytest.mark.gpu
def test_noalloc_permute_in_a_captured_graph():
    """After one eager call on the device (which resolves the scratch array's
    address), a second eager call leaves the device's free memory unchanged;
    a call captured into a HIP graph and replayed three times, on new ids
    written in place before each replay and with the workspace entry point
    run eagerly between replays, equals moe_permute_fwd on the same ids bit
    for bit every time."""
    T, k, divisor, nb, H = 2048, 8, 1, 128, 256
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(T, H, generator=g).to(BF).to(DEV)
    ids = torch.randint(-1, nb + 1, (T, k), generator=g).to(DEV)
    lib = _lib.load()
    outs = _outputs(T, k, nb, H, DEV)

    def call(stream):
        _lib.check(lib.moe_permute_fwd_noalloc(hidden.data_ptr(), T, H, ids.data_ptr(), k, divisor, nb,
                                               *(o.data_ptr() for o in outs), stream), "moe_permute_fwd_noalloc")

    call(_lib.stream_of(hidden))
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    call(_lib.stream_of(hidden))
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before, "an eager call changed the device's free memory"
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        ids.copy_(torch.randint(-1, nb + 1, (T, k), generator=g))
        graph.replay()
        torch.cuda.synchronize()
        want = _run("moe_permute_fwd", hidden, ids, divisor, nb)
        torch.cuda.synchronize()
        n = int(want[4][-1])
        for label, a, b in zip(("rows", "perm", "pos_of_slot", "counts", "offsets"), outs, want):
            if label == "rows":
                a, b = a[:n], b[:n]
            assert torch.equal(a, b), f"replay {rep}: {label}"


def test_noalloc_permute_refuses_sizes_beyond_its_scratch():
    """Host-side check only: no HIP call happens for a refused size."""
    lib = _lib.load()
    buf = ctypes.create_string_buffer(64)
    b = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    # 2**21 routes over 1024 buckets need 4096 chunks x 1025 x 4 bytes > 1 MiB
    rc = lib.moe_permute_fwd_noalloc(b, 1 << 18, 64, b, 8, 1, 1024, b, b, b, b, b, None)
    assert rc == _lib.MOE_ERR_UNSUPPORTED
    assert b"scratch" in lib.moe_last_error()
