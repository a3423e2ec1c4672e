"""The in-kernel split merge under concurrency and at the edges of its buffers
(needs an MI355X).

The last workgroup of each (KV row, head group) to finish merges the group's
split partials; it learns that it is last from an arrival counter in a slot of
library-owned counters. Each stream keeps a slot for its eager calls and each
stream capture gets one of its own, so calls that may run at the same time
never share one; calls beyond the free slots take the two-kernel merge. These
tests run captured graphs beside eager calls, more streams than slots, and
partials whose neighbouring memory holds NaN, and check every output against
the same call run alone (bit for bit) or against the oracle.
"""

import numpy as np
import pytest
import torch

import oracle
import fqkv_decode as fq

pytestmark = pytest.mark.gpu

TOL = 2e-3
DEV = "cuda"
NONE, TWO_KERNEL, DEVICE, XCD_LOCAL = 0, 1, 2, 3  # FQKV_MERGE_*


def draw(g, *shape):
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def make_call(g, Hq=32, Hkv=8, N=3000, D=128, S=24):
    q, K, V = draw(g, Hq, D).half().to(DEV), draw(g, Hkv, N, D).half().to(DEV), draw(g, Hkv, N, D).half().to(DEV)
    scratch = (torch.empty(Hq, S, device=DEV), torch.empty(Hq, S, device=DEV), torch.empty(Hq, S, D, device=DEV))
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    return q, K, V, scratch, o, S


def run(call):
    q, K, V, (mp, lp, op), o, S = call
    fq.gqa_sk_fast(q, K, V, mp, lp, op, o, S, 8, 8)


def test_graph_replays_beside_eager_calls_on_a_side_stream():
    """A captured split-K graph replayed on one stream while eager split calls
    run on another: the capture holds a slot of its own, so both stay equal
    to their solo results; afterwards solo calls on both streams are still
    exact (no counter was left behind)."""
    g = torch.Generator().manual_seed(60)
    a = make_call(g)
    b = make_call(g, Hq=64, Hkv=8, N=5000, S=32)
    run(a)
    ref_a = a[4].clone()
    run(b)
    ref_b = b[4].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(a)
    sx, sy = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (sx, sy):
        s.wait_stream(torch.cuda.current_stream())
    for _ in range(20):
        with torch.cuda.stream(sx):
            graph.replay()
        with torch.cuda.stream(sy):
            run(b)
    for s in (sx, sy):
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(a[4], ref_a)
    assert torch.equal(b[4], ref_b)
    for s in (sx, sy):
        with torch.cuda.stream(s):
            a[4].zero_()
            run(a)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        assert torch.equal(a[4], ref_a)


def test_many_captured_graphs_replay_in_turn():
    """Ten captured split-K graphs, more captures than the four slots the
    registry once reserved for them, replayed in turn for three rounds with an
    eager split call and a synchronisation between replays: every replay
    equals its call run eagerly."""
    g = torch.Generator().manual_seed(63)
    calls = [make_call(g, N=1200 + 100 * i, S=8 + i) for i in range(10)]
    alone = []
    for c in calls:
        run(c)
        alone.append(c[4].clone())
    graphs = []
    for c in calls:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run(c)
        graphs.append(graph)
    extra = make_call(g, N=900, S=12)
    run(extra)
    ref_extra = extra[4].clone()
    for _ in range(3):
        for c, graph, ref in zip(calls, graphs, alone):
            c[4].zero_()
            graph.replay()
            run(extra)
            torch.cuda.synchronize()
            assert torch.equal(c[4], ref)
            assert torch.equal(extra[4], ref_extra)


def test_more_streams_than_merge_slots():
    """Split calls in flight on 20 streams at once, more than there are eager
    slots: streams beyond them merge with the two-kernel form, and every
    output equals the same call run alone."""
    g = torch.Generator().manual_seed(61)
    calls = [make_call(g, N=1500, S=16) for _ in range(20)]
    alone = []
    for c in calls:
        run(c)
        alone.append(c[4].clone())
        c[4].zero_()
    streams = [torch.cuda.Stream() for _ in range(20)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    before = fq._ext._merge_fallback_count()
    protocols = set()
    for rep in range(3):
        for c, s in zip(calls, streams):
            with torch.cuda.stream(s):
                run(c)
            protocols.add(fq._ext._last_merge_protocol())
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for c, ref in zip(calls, alone):
        assert torch.equal(c[4], ref)
    # the streams past the eager slots were counted, and their calls took the two-kernel merge
    assert fq._ext._merge_fallback_count() > before
    # streams with a slot read a full CU mask and take the XCD-local merge (8 head groups, 16 splits)
    assert TWO_KERNEL in protocols and XCD_LOCAL in protocols and DEVICE not in protocols, protocols


@pytest.mark.parametrize("S", [5, 17, 31, 32, 40])
def test_merge_reads_stay_inside_the_partials(S, merge_mode):
    """m_part, l_part and o_part are the leading views of NaN-filled buffers,
    so any read past the last split would bring NaN (times a weight of 0
    still NaN) into the output. The output must match the oracle."""
    Hq, Hkv, N, D = 32, 8, 2500, 128
    g = torch.Generator().manual_seed(62)
    q, K, V = draw(g, Hq, D).half(), draw(g, Hkv, N, D).half(), draw(g, Hkv, N, D).half()
    nan = float("nan")
    mp = torch.full((Hq * S + 4096,), nan, device=DEV)[:Hq * S].view(Hq, S)
    lp = torch.full((Hq * S + 4096,), nan, device=DEV)[:Hq * S].view(Hq, S)
    op = torch.full((Hq * S * D + 65536,), nan, device=DEV)[:Hq * S * D].view(Hq, S, D)
    o = torch.empty(Hq, D, dtype=torch.float16, device=DEV)
    fq.gqa_sk_fast(q.to(DEV), K.to(DEV), V.to(DEV), mp, lp, op, o, S, 8, 8)
    ref = oracle.gqa_attention(q.numpy()[None], K.numpy()[None], V.numpy()[None])[0]
    out = o.float().cpu().numpy()
    assert np.isfinite(out).all()
    assert float(np.abs(out.astype(np.float64) - ref).max()) <= TOL


def test_single_block_workspace_followed_by_nan(merge_mode):
    """The C ABI's split workspace handed over as the leading bytes of a
    NaN-filled buffer: the internal split merge reads only its partials."""
    import ctypes

    L = ctypes.CDLL(fq.lib_path())
    I64, VP, SZ = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    L.fqkv_last_error.restype = ctypes.c_char_p
    L.fqkv_workspace_bytes.restype = SZ
    L.fqkv_workspace_bytes.argtypes = [I64, I64, I64, I64, ctypes.c_int, I64]
    L.fqkv_decode_attn_gqa.argtypes = [VP] * 4 + [I64] * 6 + [VP, SZ, VP]
    B, Hq, Hkv, N, D = 1, 32, 8, 9000, 128
    n = L.fqkv_workspace_bytes(B * Hkv, Hq // Hkv, N, D, 0, 8)
    assert n > 0
    g = torch.Generator().manual_seed(63)
    q, K, V = draw(g, B, Hq, D).half(), draw(g, B, Hkv, N, D).half(), draw(g, B, Hkv, N, D).half()
    buf = torch.full(((n + (1 << 20)) // 4,), float("nan"), device=DEV)  # 1 MiB of NaN after the workspace
    o = torch.empty(B, Hq, D, dtype=torch.float16, device=DEV)
    qd, Kd, Vd = q.to(DEV), K.to(DEV), V.to(DEV)
    rc = L.fqkv_decode_attn_gqa(qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), o.data_ptr(), B, Hq, Hkv, N, D, 8,
                                buf.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.fqkv_last_error().decode()
    torch.cuda.synchronize()
    out = o.float().cpu().numpy()
    assert np.isfinite(out).all()
    ref = oracle.gqa_attention(q.numpy(), K.numpy(), V.numpy())
    assert float(np.abs(out.astype(np.float64) - ref).max()) <= TOL


@pytest.mark.parametrize("Hkv,N,D,S", [(8, 16384, 128, 32), (8, 512, 128, 16), (64, 4096, 128, 16),
                                       (8, 8192, 64, 32), (4, 2048, 128, 16)])
def test_xcd_local_merge_alternating_inputs(Hkv, N, D, S):
    """With 16 or more splits and a multiple of 8 (KV row, head group) pairs,
    every split of a group runs on one XCD and the merge meets in that XCD's
    L2 (8 and 64 groups here); 4 groups keep the device-scope protocol. Two
    inputs alternate through one scratch buffer six times: each output equals
    its first result bit for bit (a merge reading the other input's stale
    partials would not), the partials equal the two-kernel merge's bit for bit,
    and the output agrees with the oracle."""
    g = torch.Generator().manual_seed(Hkv * 1000 + N + S)
    Hq = 4 * Hkv
    a = make_call(g, Hq=Hq, Hkv=Hkv, N=N, D=D, S=S)
    b = make_call(g, Hq=Hq, Hkv=Hkv, N=N, D=D, S=S)
    scratch, o = a[3], a[4]
    b = b[:3] + (scratch, o, S)
    first = {}
    # 4 query heads per KV row make one head group per row: Hkv groups
    expect = XCD_LOCAL if Hkv % 8 == 0 else DEVICE
    for i in range(12):
        c = (a, b)[i % 2]
        run(c)
        assert fq._ext._last_merge_protocol() == expect, (i, fq._ext._last_merge_protocol())
        torch.cuda.synchronize()
        if i < 2:
            first[i] = (o.clone(), scratch[2].clone())
        else:
            assert torch.equal(o, first[i % 2][0]), f"call {i}"
    fq._ext._set_two_kernel_merge(True)
    try:
        for i in (0, 1):
            run((a, b)[i])
            assert fq._ext._last_merge_protocol() == TWO_KERNEL
            torch.cuda.synchronize()
            assert torch.equal(scratch[2], first[i][1]), f"partials of input {i}"
    finally:
        fq._ext._set_two_kernel_merge(False)
    for i, c in enumerate((a, b)):
        q, K, V = (x.cpu().double().numpy() for x in c[:3])
        ref = oracle.gqa_attention(q[None], K[None], V[None])[0]
        err = np.abs(first[i][0].cpu().double().numpy() - ref).max()
        assert err <= TOL, (i, err)


def test_xcd_probe_found_the_round_robin_order():
    """MI355X deals a launch's workgroups to its 8 XCDs in turn; the probe that
    the first eager split call ran must have found exactly that period."""
    g = torch.Generator().manual_seed(65)
    run(make_call(g, N=4096, S=32))
    torch.cuda.synchronize()
    assert fq._ext._xcd_period(torch.cuda.current_device()) == 8


def test_forked_streams_in_one_capture_take_separate_slots():
    """Two split calls captured on forked streams of one graph (the side
    stream joins the capture through an event wait, so both report the same
    capture id) run side by side on replay; each must have its own arrival
    counters. Every replay equals the eager results bit for bit."""
    g = torch.Generator().manual_seed(66)
    a = make_call(g, N=6000, S=32)
    b = make_call(g, N=7000, S=32)
    run(a)
    ref_a = a[4].clone()
    run(b)
    ref_b = b[4].clone()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cur = torch.cuda.current_stream()
        side.wait_stream(cur)
        run(a)
        with torch.cuda.stream(side):
            run(b)
        cur.wait_stream(side)
    for _ in range(10):
        a[4].zero_()
        b[4].zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a[4], ref_a)
        assert torch.equal(b[4], ref_b)
    # eager calls afterwards are unaffected
    run(a)
    torch.cuda.synchronize()
    assert torch.equal(a[4], ref_a)


def test_cu_masked_stream_keeps_the_device_scope_merge():
    """A stream created with a CU mask that leaves half the CUs out may deal
    workgroups to the XCDs in another order, so its split calls take the
    device-scope merge; the output equals an unmasked stream's bit for bit."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    L = ctypes.CDLL(fq.lib_path())
    VP, I64 = ctypes.c_void_p, ctypes.c_int64
    L.fqkv_gqa_sk_fast.argtypes = [VP] * 7 + [I64] * 7 + [VP]
    L.fqkv_last_error.restype = ctypes.c_char_p
    g = torch.Generator().manual_seed(67)
    Hq, Hkv, N, D, S = 32, 8, 8192, 128, 32
    q, K, V, (mp, lp, op), o, _ = make_call(g, Hq=Hq, Hkv=Hkv, N=N, D=D, S=S)
    args = [x.data_ptr() for x in (q, K, V, mp, lp, op, o)] + [Hq, Hkv, N, D, S, 8, 8]
    torch.cuda.synchronize()
    assert L.fqkv_gqa_sk_fast(*args, torch.cuda.current_stream().cuda_stream) == 0, L.fqkv_last_error()
    assert L.fqkv_last_merge_protocol() == XCD_LOCAL
    torch.cuda.synchronize()
    ref = o.clone()
    words = (fq._ext._cu_count() + 31) // 32
    mask = (ctypes.c_uint32 * words)(*([0x55555555] * words))
    st = ctypes.c_void_p()
    rc = hip.hipExtStreamCreateWithCUMask(ctypes.byref(st), ctypes.c_uint32(words), mask)
    if rc != 0:
        # a CU-masked stream needs a hardware queue of its own; a runtime limited
        # to a few queues per process (GPU_MAX_HW_QUEUES) refuses one. The refusal
        # stays pending as HIP's last error, which the next HIP call would report.
        hip.hipGetLastError()
        assert hip.hipGetLastError() == 0
        pytest.skip("hipExtStreamCreateWithCUMask failed with HIP error %d on this system" % rc)
    try:
        for _ in range(3):
            o.zero_()
            torch.cuda.synchronize()
            assert L.fqkv_gqa_sk_fast(*args, st) == 0, L.fqkv_last_error()
            assert L.fqkv_last_merge_protocol() == DEVICE
            assert hip.hipStreamSynchronize(st) == 0
            assert torch.equal(o, ref)
    finally:
        hip.hipStreamDestroy(st)
