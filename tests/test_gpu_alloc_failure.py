"""Failed device allocations and a full page pool: a call that cannot get the
memory it needs returns NDA_ERR_NOMEM and changes no session state.

An allocator installed through nda_set_allocator (the counterpart of the
engine's ND_ALLOC / ND_FREE seams, engine/include/nd_model.h:35-68) wraps
hipMalloc and refuses requests while armed. The failure is forced from the
host; every kernel that runs still gets valid memory. After each refused call
the test checks that positions and device bytes are as before, that the page
pool lost nothing (it is filled to its last page afterwards), and that the
same call then succeeds with outputs matching the oracle."""
import sys

import numpy as np
import pytest

import ndoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
NOMEM = -2


def nda():
    import ndattn
    return ndattn


def say(*a):
    print("[gpu-case]", *a, flush=True)
    sys.stdout.flush()


def _states(ctx, seqs):
    return [ctx.seq_state(b) for b in seqs]


def _pages(n, P):
    return (n + P - 1) // P


def _fill_pool(N, ctx, seqs, P, per_seq, npages):
    """Take exactly `npages` pages with empty sequences `seqs` (at most
    per_seq each, one window): all must be granted, and one page more then
    refused."""
    left, taken = npages, {}
    for s in seqs:
        taken[s] = min(left, per_seq)
        if taken[s]:
            ctx.seq_reserve(s, taken[s] * P)
        left -= taken[s]
    assert left == 0, "not enough empty sequences to fill the pool"
    s = next(s for s in seqs if taken[s] < per_seq)
    with pytest.raises(N.NdaError) as e:
        ctx.seq_reserve(s, (taken[s] + 1) * P)
    assert e.value.code == NOMEM


def test_refused_buffer_growth_changes_nothing(allocator):
    """A prefill whose row staging and work list must grow, a split decode
    whose partials must grow, and an inspection write whose staging must
    grow, each with every allocation refused: NDA_ERR_NOMEM, positions and
    device bytes unchanged, no page taken, and the buffers the context had
    still serve calls that fit them. Then the same prefill succeeds."""
    N = nda()
    nh, d, P, W = 8, 64, 16, 2048
    B = 20
    rng = np.random.default_rng(41)
    hist = [int(x) for x in rng.integers(100, 1500, B)]
    SPARE = 360                                  # pages left free after the setup below
    setup_pages = sum(_pages(L + (1 if b in (0, 1, 2, 3, 5, 6) else 0), P) for b, L in enumerate(hist))
    total = setup_pages + SPARE
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B + 3, max_pages=total, split_chunk=256)
    for b, L in enumerate(hist):
        kf = rng.standard_normal((L, nh, d)).astype(np.float32)
        vf = rng.standard_normal((L, nh, d)).astype(np.float32)
        ctx.kv_write(0, b, 0, O.f32_to_f16_bits(kf), O.f32_to_f16_bits(vf))
        ctx.seq_set_pos(b, L)
    # small prefills size the staging buffers
    one = [N.DevBuf(4 * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(one[:3]):
        bb.fill_normal(4 * nh * d, 0, 10 + i)
    ctx.prefill(0, [1] * 4, *one[:3], one[3], seq_ids=[0, 1, 2, 3])
    ctx.sync()
    ctx.advance(4, [0, 1, 2, 3], 1)

    # more rows than the row staging's first size (4096) holds
    ntok = [int(x) for x in rng.integers(215, 240, B)]
    T = sum(ntok)
    q = rng.standard_normal((T, nh, d)).astype(np.float32)
    kv = rng.standard_normal((T, nh, d)).astype(np.float32)
    dq, dk = N.DevBuf.from_array(q), N.DevBuf.from_array(kv)
    dout = N.DevBuf(T * nh * d * 4)
    seqs = list(range(B))
    before, dev_bytes = _states(ctx, seqs), ctx.device_bytes

    say("prefill of", T, "rows, allocations refused")
    allocator.armed = True
    with pytest.raises(N.NdaError) as e:
        ctx.prefill(0, ntok, dq, dk, dk, dout)
    allocator.armed = False
    assert e.value.code == NOMEM and allocator.refused >= 1
    assert _states(ctx, seqs) == before and ctx.device_bytes == dev_bytes

    say("the kept staging serves a call that fits it")
    ctx.prefill(0, [1, 1], *one[:3], one[3], seq_ids=[5, 6])
    ctx.sync()
    ctx.advance(2, [5, 6], 1)
    before = _states(ctx, seqs)

    say("split decode step, partials refused")
    qd = N.DevBuf(B * nh * d * 4)
    qd.fill_normal(B * nh * d, 0, 30)
    outd = N.DevBuf(B * nh * d * 4)
    allocator.armed = True
    with pytest.raises(N.NdaError) as e:
        ctx.step(0, B, qd, qd, qd, outd)
    allocator.armed = False
    assert e.value.code == NOMEM
    assert _states(ctx, seqs) == before and ctx.device_bytes == dev_bytes

    say("inspection write, staging refused")
    kw = O.f32_to_f16_bits(rng.standard_normal((1800, nh, d)).astype(np.float32))
    allocator.armed = True
    with pytest.raises(N.NdaError) as e:
        ctx.kv_write(0, B, 0, kw, kw)
    allocator.armed = False
    assert e.value.code == NOMEM
    assert ctx.seq_state(B) == (0, 0, -1) and ctx.device_bytes == dev_bytes

    say("no page was lost: the", SPARE, "spare pages are all free")
    _fill_pool(N, ctx, [B, B + 1, B + 2], P, W // P, SPARE)
    for s in (B, B + 1, B + 2):
        ctx.seq_reset(s)

    say("the refused prefill, now with memory")
    ctx.prefill(0, ntok, dq, dk, dk, dout)
    ctx.sync()
    got = dout.to_array(np.float32, (T, nh * d))
    worst, r = 0.0, 0
    for b in range(B):
        pos0 = before[b][0]
        end = pos0 + ntok[b]
        kk, vv, _, _ = ctx.kv_read(0, b, 0, end)
        for t in range(ntok[b]):
            if t in (0, ntok[b] - 1):
                view = O.kv_view(kk, vv, None, None, nh, end, 0, pos0 + t, O.KV_F16)
                worst = max(worst, float(np.abs(got[r] - O.attend_view(view, q[r].ravel())).max()))
            r += 1
    say("worst", worst)
    assert worst <= TOL
    ctx.close()


def test_full_pool_part_way_gives_pages_back(allocator):
    """A prefill whose last sequence does not fit the page pool after the
    others took theirs: NDA_ERR_NOMEM, and every page goes back."""
    N = nda()
    nh, d, P, W = 8, 64, 16, 512
    B, total = 6, 40
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_INT8, max_seqs=B + 2, max_pages=total)
    ntok = [64, 64, 64, 200, 200, 64]       # 4 + 4 + 4 + 13 + 13 + 4 = 42 pages of 40
    T = sum(ntok)
    bufs = [N.DevBuf(T * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(bufs[:3]):
        bb.fill_normal(T * nh * d, 0, 20 + i)
    with pytest.raises(N.NdaError) as e:
        ctx.prefill(0, ntok, *bufs[:3], bufs[3])
    assert e.value.code == NOMEM
    assert _states(ctx, range(B)) == [(0, 0, -1)] * B
    _fill_pool(N, ctx, [B, B + 1], P, W // P, total)
    ctx.close()


def test_attach_without_room_for_the_ring_tail(allocator):
    """Attaching to a prefix longer than the sink clamp copies its tail into
    the sequence's ring; without pages for it the attach is refused before
    the sequence changes. Once pages are freed it succeeds."""
    N = nda()
    nh, d, P, W = 8, 64, 16, 96
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_INT8, max_seqs=3, max_pages=12)
    n = 80                       # sink clamp 96 - 64 = 32: a 48-position (3-page) tail
    bufs = [N.DevBuf(n * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(bufs[:3]):
        bb.fill_normal(n * nh * d, 0, 40 + i)
    ctx.prefill(0, [n], *bufs[:3], bufs[3], seq_ids=[0])
    ctx.advance(1, [0], n)
    pid = ctx.prefix_build(0)    # 5 pages for the sequence, 5 for the prefix: 2 free
    with pytest.raises(N.NdaError) as e:
        ctx.seq_attach(1, pid)
    assert e.value.code == NOMEM
    assert ctx.seq_state(1) == (0, 0, -1)
    ctx.seq_reset(0)
    ctx.seq_attach(1, pid)
    assert ctx.seq_state(1)[2] == pid
    ctx.seq_reset(1)
    ctx.prefix_free(pid)
    ctx.close()


def test_front_init_all_or_nothing(allocator):
    """nda_front_init refused part-way frees what it took; a retry works."""
    N = nda()
    ctx = N.Context(1, 8, 8, 64, 64, 128, kv_dtype=O.KV_INT8, max_seqs=4)
    dev_bytes = ctx.device_bytes
    allocator.seen = 0
    allocator.refuse_nth = 3             # the third of its six buffers
    with pytest.raises(N.NdaError) as e:
        ctx.front_init(3, 10000.0)
    assert e.value.code == NOMEM and allocator.refused == 1 and ctx.device_bytes == dev_bytes
    allocator.refuse_nth = 0
    ctx.front_init(3, 10000.0)
    assert ctx.device_bytes > dev_bytes
    ctx.close()


def test_two_launch_step_refused_before_its_append(allocator):
    """nda_step on a batch whose decode takes the shared-prefix pass (1024
    sequences on one 213-token prefix) runs the append and the decode as
    two launches. With the decode's partials refused, the call fails before
    the append: the position is still unstored, positions and device bytes
    are as before. Then the same step succeeds and meets the oracle."""
    N = nda()
    nh, d, W, B, npre = 8, 64, 384, 1024, 213
    ctx = N.Context(1, nh, nh, d, d, W, kv_dtype=O.KV_F16, max_seqs=B + 1)
    bufs = [N.DevBuf(npre * nh * d * 4) for _ in range(4)]
    for i, bb in enumerate(bufs[:3]):
        bb.fill_normal(npre * nh * d, 0, 60 + i)
    ctx.prefill(0, [npre], bufs[0], bufs[1], bufs[2], bufs[3], seq_ids=[B])
    ctx.advance(1, [B], npre)
    pid = ctx.prefix_build(B)
    for b in range(B):
        ctx.seq_attach(b, pid)
    ctx.sync()
    q, k, v, out = (N.DevBuf(B * nh * d * 4) for _ in range(4))
    for i, bb in enumerate((q, k, v)):
        bb.fill_normal(B * nh * d, 0, 70 + i)
    seqs = list(range(B))
    before, dev_bytes = _states(ctx, seqs), ctx.device_bytes
    say("shared-prefix step of", B, "sequences, allocations refused")
    allocator.armed = True
    with pytest.raises(N.NdaError) as e:
        ctx.step(0, B, q, k, v, out)
    allocator.armed = False
    assert e.value.code == NOMEM and allocator.refused >= 1
    assert _states(ctx, seqs) == before and ctx.device_bytes == dev_bytes
    for b in (0, B - 1):
        with pytest.raises(N.NdaError) as e:
            ctx.kv_read(0, b, npre, 1)         # the refused step stored nothing
        assert e.value.code == -4
    say("the same step with memory")
    ctx.step(0, B, q, k, v, out)
    ctx.sync()
    qh = q.to_array(np.float32, (B, nh * d))
    got = out.to_array(np.float32, (B, nh * d))
    worst = 0.0
    for b in (0, 517, B - 1):
        kk, vv, _, _ = ctx.kv_read(0, b, 0, npre + 1)
        view = O.kv_view(kk, vv, None, None, nh, npre + 1, 0, npre, O.KV_F16)
        worst = max(worst, float(np.abs(got[b] - O.attend_view(view, qh[b])).max()))
    say("worst", worst)
    assert worst <= TOL
    for b in range(B + 1):
        ctx.seq_reset(b)
    ctx.prefix_free(pid)
    ctx.close()
