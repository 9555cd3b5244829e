"""Many-group batches from two host threads at once, each on its own stream (needs an MI355X).

A batch whose input-select pairs span two dtype groups runs one group's pivot
and capture launches on the library's side stream, and every batch call
uploads its table through the library's pinned staging buffer.  Both are
shared by all the calls on a device.  Calls made from two threads and
streams at once must give the same records, bit for bit, as the same batches
made one after another; a record that read the other call's table or work
lists would not.
"""

import sys
import threading

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _batch(seed: int, count: int = 300):
    """fp32 and bf16 pairs of 9 K to 40 K elements (more large pairs than the device has CUs)."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    sizes = torch.randint(9_000, 40_000, (count,), generator=gen, device=DEV).tolist()
    pairs = []
    for i, n in enumerate(sizes):
        r = torch.randn(n, generator=gen, device=DEV)
        g = r + 1e-6 * torch.randn(n, generator=gen, device=DEV)
        if i % 2:
            g, r = g.to(torch.bfloat16), r.to(torch.bfloat16)
        pairs.append((g, r))
    return pairs


def _diff(a: dict, b: dict) -> dict:
    """The fields of two records that differ (NaN equals NaN)."""
    return {f: (a[f], b[f]) for f in a if not (a[f] == b[f] or (a[f] != a[f] and b[f] != b[f]))}


def test_concurrent_batches_match_sequential_ones():
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    from kernelverse_amd import _lib, verdict
    _lib.load()
    batches = [_batch(71), _batch(72)]
    torch.cuda.synchronize()
    _say("batch threads: sequential reference records")
    want = [verdict.verdict_records(b) for b in batches]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = [[], []]
    errors = []

    def run(k: int):
        try:
            with torch.cuda.stream(streams[k]):
                for _ in range(6):
                    got[k].append(verdict.verdict_records(batches[k]))
        except Exception as e:  # noqa: BLE001 -- reported by the main thread
            errors.append((k, repr(e)))

    _say("batch threads: two threads, six batches each")
    threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=240)
    assert not any(t.is_alive() for t in threads), "a batch thread did not finish"
    assert not errors, errors
    for k in range(2):
        assert len(got[k]) == 6
        for it, recs in enumerate(got[k]):
            for i, (a, b) in enumerate(zip(recs, want[k])):
                d = _diff(a, b)
                assert not d, (k, it, i, d)
    verdict.release_buffers()


def test_batch_refuses_a_capturing_stream():
    """kvv_verdict_batch on a stream that is being captured into a graph returns
    KVV_E_UNSUPPORTED and enqueues nothing (a replay would reuse a stale upload of
    its pair table); the capture itself goes on and replays normally."""
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: the gpu tests must run on the MI355X box")
    import ctypes
    from kernelverse_amd import _lib, verdict
    lib = _lib.load()
    pairs = _batch(73, count=8)
    jobs = [verdict._Job(g, r, f"o{i}", None, None, verdict.MAX_SAMPLES) for i, (g, r) in enumerate(pairs)]
    n = len(jobs)
    views = [verdict._device_views(g, r) for g, r in pairs]
    gts = (_lib.KvvTensor * n)(*[v[0] for v in views])
    rts = (_lib.KvvTensor * n)(*[v[1] for v in views])
    pols = (_lib.KvvPolicy * n)(*[j.kpolicy for j in jobs])
    size = ctypes.c_size_t()
    _lib.check(lib.kvv_batch_workspace_size(n, gts, rts, pols, ctypes.byref(size)), "kvv_batch_workspace_size")
    ws = torch.empty(size.value, dtype=torch.uint8, device=DEV)
    out = torch.zeros(n * ctypes.sizeof(_lib.KvvResult), dtype=torch.uint8, device=DEV)
    x = torch.zeros(4, device=DEV)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    _say("batch capture: kvv_verdict_batch inside a capture")
    with torch.cuda.graph(graph):
        rc = lib.kvv_verdict_batch(n, gts, rts, pols, out.data_ptr(), ws.data_ptr(), size.value,
                                   torch.cuda.current_stream().cuda_stream)
        x.add_(1.0)
    assert rc == -4, rc  # KVV_E_UNSUPPORTED
    assert b"captured" in lib.kvv_last_error()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), torch.ones(4))
    assert int(out.sum().item()) == 0  # nothing of the batch ran
    # the same call outside a capture runs
    _lib.check(lib.kvv_verdict_batch(n, gts, rts, pols, out.data_ptr(), ws.data_ptr(), size.value,
                                     torch.cuda.current_stream().cuda_stream), "kvv_verdict_batch")
    torch.cuda.synchronize()
    assert int(out.sum().item()) != 0
