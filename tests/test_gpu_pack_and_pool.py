"""Step packing (bit-exact) and device page operations, through the C ABI."""
import numpy as np
import pytest

import workloads

pytestmark = pytest.mark.gpu


def expected_packing(step):
    """Concatenation of each row's AsSpan() cut to ceil(total/16), and per-query totals."""
    rows = [0]
    ids = []
    ctxs = []
    for b in range(step.num_rows):
        ql = int(step.lens[b])
        pos = int(step.positions[b])
        tc = int(step.token_counts[b])
        last = min(tc, pos + ql) if ql > 0 else 0
        pages = -(-last // 16)
        ids.extend(step.table(b)[:pages].tolist())
        rows.append(len(ids))
        ctxs.extend(min(tc, pos + i + 1) for i in range(ql))
    return np.array(rows, np.int32), np.array(ids, np.int32), np.array(ctxs, np.int32)


@pytest.mark.parametrize("which", ["ragged", "prefill", "llama8b"])
def test_packing_is_bit_exact(gsp, ctx, which):
    if which == "ragged":
        step = workloads.small_step(seed=1, rows=40, n_heads=8, n_kv=2, head_dim=64, ctx_hi=700, total_blocks=4096)
        # Tables longer than needed (BlockTable spans grow ahead of pos): extra ids must not be packed.
        step.positions = np.maximum(step.positions - 20, 0).astype(np.int32)
    elif which == "prefill":
        step = workloads.small_step(seed=2, rows=7, n_heads=8, n_kv=2, head_dim=64, ctx_hi=300, total_blocks=512,
                                    q_lens=np.array([1, 9, 1, 33, 0, 2, 16], np.int32))
    else:
        step = workloads.llama8b_decode(steps=300)
    # Packing reads only the pool's geometry; a thin pool of the same block count will do.
    pool = gsp.Pool.create(ctx, total_blocks=step.total_blocks, layers=1, heads_kv=step.n_kv, head_dim=4)
    info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                         q_lens=step.q_lens)
    pool.destroy()
    rows, ids, ctxs = ctx.download_step()
    er, ei, ec = expected_packing(step)
    assert np.array_equal(rows, er)
    assert np.array_equal(ids, ei)
    assert np.array_equal(ctxs, ec)
    assert info.total_q == step.total_q
    assert info.kv_tokens == step.kv_tokens()


def test_pack_rejects_what_the_reference_throws_on(gsp, ctx):
    pool = gsp.Pool.create(ctx, total_blocks=4, layers=1, heads_kv=1, head_dim=4)
    ok = dict(positions=[3], token_counts=[4], bt_offsets=[0, 1], bt_ids=[0], max_seq_len=16)

    def pack(**kw):
        a = dict(ok)
        a.update(kw)
        ctx.pack_step(pool, **a)

    pack()
    for bad in (dict(positions=[16]), dict(positions=[-1]), dict(max_seq_len=0), dict(token_counts=[17]),
                dict(token_counts=[-1]), dict(positions=[40], token_counts=[41], max_seq_len=64),
                dict(bt_ids=[-3]), dict(bt_ids=[4]), dict(positions=[10], q_lens=[7]),
                # CSR offsets outside the caller's id array, negative or decreasing: refused
                # before any id is read (the array's length travels as n_bt_ids).
                dict(bt_offsets=[0, 2]), dict(bt_offsets=[1, 2], bt_ids=[0, 0], n_bt_ids=1),
                dict(bt_offsets=[-1, 1]), dict(bt_offsets=[1, 0]), dict(n_bt_ids=-1)):
        with pytest.raises(gsp.InvalidArgument):
            pack(**bad)
    # After a failed pack there is no step to run.
    with pytest.raises(gsp.StateError):
        ctx.step_info()
    pool.destroy()


def test_attention_rejects_ids_outside_the_pool(torch_mod, gsp, ctx):
    torch = torch_mod
    k = torch.zeros((4, 1, 1, 16, 64), device="cuda")
    pool = gsp.Pool.wrap(ctx, k.data_ptr(), k.data_ptr(), 4, 1, 1, 64)
    k2 = torch.zeros((2, 1, 2, 16, 64), device="cuda")
    pool2 = gsp.Pool.wrap(ctx, k2.data_ptr(), k2.data_ptr(), 2, 1, 2, 64)
    with pytest.raises(gsp.InvalidArgument):  # block id 4 of a 4-block pool
        ctx.pack_step(pool, [0], [1], [0, 1], [4], 16)
    q = torch.zeros((1, 2, 64), device="cuda")
    ctx.pack_step(pool, [0], [1], [0, 1], [3], 16)
    with pytest.raises(gsp.InvalidArgument):  # layer outside the pool
        ctx.attention_step(pool, 1, 1, q.data_ptr(), q.data_ptr(), 0.125)
    with pytest.raises(gsp.InvalidArgument):  # packed for another pool geometry
        ctx.attention_step(pool2, 0, 2, q.data_ptr(), q.data_ptr(), 0.125)
    pool2.destroy()
    # (Groups above 16 run as tiles of 16 heads: tests/test_gpu_shapes.py.)
    ctx.set_decode_path(gsp.DECODE_DPP)
    try:
        with pytest.raises(gsp.Unsupported):  # the DPP kernel stops at 8
            ctx.attention_step(pool, 0, 9, q.data_ptr(), q.data_ptr(), 0.125)
    finally:
        ctx.set_decode_path(gsp.DECODE_AUTO)
    pool.destroy()


def test_store_layout_exact(torch_mod, gsp, ctx):
    """PagedAttentionTests.cs:81-109: Store(layer 1, slot 2) lands at GetKeyPtr(b, 1, h, 2)."""
    torch = torch_mod
    pool = gsp.Pool.create(ctx, total_blocks=4, layers=2, heads_kv=2, head_dim=4)
    alloc = gsp.BlockAllocator(4)
    ok, blk = alloc.try_allocate_block()
    assert ok
    k = torch.tensor([[1, 2, 3, 4, 5, 6, 7, 8]], dtype=torch.float32, device="cuda")
    v = torch.tensor([[10, 20, 30, 40, 50, 60, 70, 80]], dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    pool.write_tokens(1, [blk], [2], k.data_ptr(), v.data_ptr())
    ctx.sync()
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(np.float32).reshape(4, 2, 2, 16, 4)
    V = pool.download(1, vb).view(np.float32).reshape(4, 2, 2, 16, 4)
    assert np.array_equal(K[blk, 1, 0, 2], [1, 2, 3, 4]) and np.array_equal(K[blk, 1, 1, 2], [5, 6, 7, 8])
    assert np.array_equal(V[blk, 1, 0, 2], [10, 20, 30, 40]) and np.array_equal(V[blk, 1, 1, 2], [50, 60, 70, 80])
    mask = np.ones(K.shape, bool)
    mask[blk, 1, :, 2] = False
    assert not K[mask].any() and not V[mask].any()  # pools start zeroed and nothing else was written
    pool.destroy()


def test_store_fp16_rounds_to_nearest_even(torch_mod, gsp, ctx):
    torch = torch_mod
    rng = np.random.default_rng(0)
    n, hkv, d = 37, 8, 128
    kh = (rng.standard_normal((n, hkv, d)) * 3).astype(np.float32)
    vh = (rng.standard_normal((n, hkv, d)) * 1e-3).astype(np.float32)
    pool = gsp.Pool.create(ctx, total_blocks=8, layers=1, heads_kv=hkv, head_dim=d, kv_dtype=gsp.KV_F16)
    blocks = np.repeat(np.arange(3), 16)[:n]
    slots = np.tile(np.arange(16), 3)[:n]
    kd = torch.from_numpy(kh).cuda()
    vd = torch.from_numpy(vh).cuda()
    torch.cuda.synchronize()
    pool.write_tokens(0, blocks, slots, kd.data_ptr(), vd.data_ptr())
    ctx.sync()
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(np.float16).reshape(8, 1, hkv, 16, d)
    V = pool.download(1, vb).view(np.float16).reshape(8, 1, hkv, 16, d)
    for i in range(n):
        assert np.array_equal(K[blocks[i], 0, :, slots[i]].view(np.uint16), kh[i].astype(np.float16).view(np.uint16))
        assert np.array_equal(V[blocks[i], 0, :, slots[i]].view(np.uint16), vh[i].astype(np.float16).view(np.uint16))
    with pytest.raises(gsp.InvalidArgument):
        pool.write_tokens(0, [8], [0], kd.data_ptr(), vd.data_ptr())
    with pytest.raises(gsp.InvalidArgument):
        pool.write_tokens(0, [0], [16], kd.data_ptr(), vd.data_ptr())
    pool.destroy()


def test_cow_fork_copies_page_on_device(torch_mod, gsp, ctx):
    """PrefixHashKvCacheTests.cs:134-181 with a device pool attached to the allocator."""
    torch = torch_mod
    pool = gsp.Pool.create(ctx, total_blocks=16, layers=2, heads_kv=2, head_dim=32)
    alloc = gsp.BlockAllocator(16)
    alloc.attach_pool(ctx, pool)
    ta = gsp.BlockTable(alloc)
    assert ta.append_tokens(10) == 10
    shared = ta.get_block_id(0)
    # Sentinel 42.0 at (shared, layer 0, head 0, slot 0) and a distinct value per slot elsewhere.
    k = torch.arange(10 * 2 * 32, dtype=torch.float32, device="cuda").reshape(10, 2, 32)
    k[0, 0, 0] = 42.0
    torch.cuda.synchronize()
    for layer in (0, 1):
        pool.write_tokens(layer, [shared] * 10, list(range(10)), k.data_ptr(), k.data_ptr())
    pool.copy_block_data(shared, shared, 0)  # valid_tokens <= 0 is a no-op
    tb = gsp.BlockTable(alloc)
    alloc.retain_block(shared)
    tb.attach_prefix_blocks([shared], 10)
    ok, forked, off = ta.append_token()  # shared partial page -> fork
    assert ok and off == 10 and forked != shared
    ctx.sync()
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(np.float32).reshape(16, 2, 2, 16, 32)
    V = pool.download(1, vb).view(np.float32).reshape(16, 2, 2, 16, 32)
    assert K[forked, 0, 0, 0, 0] == 42.0
    assert np.array_equal(K[forked, :, :, :10], K[shared, :, :, :10])
    assert np.array_equal(V[forked, :, :, :10], V[shared, :, :, :10])
    assert not K[forked, :, :, 10:].any()  # only the valid tokens are copied
    # Mutating the fork leaves the shared page alone.
    z = torch.full((1, 2, 32), 999.0, device="cuda")
    torch.cuda.synchronize()
    pool.write_tokens(0, [forked], [0], z.data_ptr(), z.data_ptr())
    ctx.sync()
    K = pool.download(0, kb).view(np.float32).reshape(16, 2, 2, 16, 32)
    assert K[forked, 0, 0, 0, 0] == 999.0 and K[shared, 0, 0, 0, 0] == 42.0
    ta.release_all()
    tb.release_all()
    assert alloc.free_blocks_count == 16
    alloc.attach_pool(None, None)
    pool.destroy()


def test_back_to_back_packs_without_host_sync(torch_mod, gsp, ctx):
    """Packs alternate between two device slots, each uploaded by one copy kernel on
    the context's stream: a pack may overwrite a slot only after the kernels of the
    step packed two calls earlier have read it.  Nine packs of three different steps,
    each followed by its attention and its KV write, with no host sync between
    them: every output must match the oracle."""
    from gpu_helpers import TOL, max_err, oracle_step, to_device_pool

    torch = torch_mod
    base = workloads.small_step(seed=61, rows=24, n_heads=28, n_kv=4, head_dim=128, ctx_lo=40, ctx_hi=600,
                                total_blocks=1024)
    steps = [base.subset(np.arange(0, 24))[0], base.subset(np.arange(3, 10))[0], base.subset(np.arange(10, 24, 2))[0]]
    q, k, v = workloads.host_values(base, layers=2)
    pool, keep = to_device_pool(torch, gsp, ctx, base, k, v)
    qs = [torch.from_numpy(np.ascontiguousarray(q[: s.total_q])).cuda() for s in steps]
    outs = [torch.full((s.total_q, s.n_heads, s.head_dim), float("nan"), device="cuda") for s in steps for _ in
            range(3)]
    kn = torch.zeros((24, 4, 128), device="cuda")
    torch.cuda.synchronize()
    try:
        for i in range(9):
            s = steps[i % 3]
            ctx.set_split_pages(2 + i % 3)  # different schedules, different step sizes
            ctx.pack_step(pool, s.positions, s.token_counts, s.bt_offsets, s.bt_ids, s.max_seq_len, want_info=False)
            ctx.attention_step(pool, 0, s.n_heads, qs[i % 3].data_ptr(), outs[(i % 3) * 3 + i // 3].data_ptr(),
                               s.scale)
            pool.write_step(1, kn.data_ptr(), kn.data_ptr())  # layer 1: attention reads layer 0
        ctx.set_split_pages(0)
        ctx.sync()
        for j, s in enumerate(steps):
            ref = oracle_step(s, q[: s.total_q], k, v)
            for r in range(3):
                assert max_err(outs[j * 3 + r].cpu().numpy(), ref) <= TOL["f32"], f"step {j} repeat {r}"
    finally:
        ctx.set_split_pages(0)
        pool.destroy()


def test_concurrent_cow_forks_copy_pages_on_device(torch_mod, gsp, ctx):
    """PrefixHashKvCacheAdversarialTests.cs:43-107 with the pages on the device: 16
    sequences share one block holding tokens 0..7 and append token 8 at once from 16
    threads.  Each fork copies the shared page on the device; afterwards every
    sequence's page holds the prefix tokens and its own token 8."""
    import threading

    torch = torch_mod
    nkv, d = 1, 16
    pool = gsp.Pool.create(ctx, total_blocks=64, layers=1, heads_kv=nkv, head_dim=d)
    alloc = gsp.BlockAllocator(64)
    alloc.attach_pool(ctx, pool)
    ok, shared = alloc.try_allocate_block()
    assert ok
    prefix = torch.arange(8 * d, dtype=torch.float32, device="cuda").reshape(8, nkv, d) + 100.0
    torch.cuda.synchronize()
    pool.write_tokens(0, [shared] * 8, list(range(8)), prefix.data_ptr(), prefix.data_ptr())
    ctx.sync()
    for _ in range(15):
        alloc.retain_block(shared)
    tables = [gsp.BlockTable(alloc) for _ in range(16)]
    for t in tables:
        t.attach_prefix_blocks([shared], 8)
    got = [None] * 16
    barrier = threading.Barrier(16)

    def one(i):
        barrier.wait()
        got[i] = tables[i].append_token()

    threads = [threading.Thread(target=one, args=(i,)) for i in range(16)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    ctx.sync()
    ids = [g[1] for g in got]
    assert all(g[0] and g[2] == 8 for g in got) and len(set(ids)) == 16
    marks = torch.stack([torch.full((nkv, d), 1000.0 + i, device="cuda") for i in range(16)])
    torch.cuda.synchronize()
    pool.write_tokens(0, ids, [8] * 16, marks.data_ptr(), marks.data_ptr())
    ctx.sync()
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(np.float32).reshape(64, 1, nkv, 16, d)
    V = pool.download(1, vb).view(np.float32).reshape(64, 1, nkv, 16, d)
    want = prefix.cpu().numpy()
    for i, b in enumerate(ids):
        assert np.array_equal(K[b, 0, :, :8].transpose(1, 0, 2), want), f"sequence {i}: prefix of block {b}"
        assert np.array_equal(V[b, 0, :, :8].transpose(1, 0, 2), want)
        assert np.all(K[b, 0, :, 8] == 1000.0 + i) and np.all(V[b, 0, :, 8] == 1000.0 + i)
    for t in tables:
        t.release_all()
    assert alloc.free_blocks_count == 64
    alloc.attach_pool(None, None)
    pool.destroy()


def test_step_upload_through_growing_staging(gsp):
    """A fresh context packs steps whose images grow and shrink, so that each slot's pinned
    buffer is reallocated (and its device address looked up again) while the other slot
    holds the previous step; every upload is checked bit for bit by downloading it."""
    ctx2 = gsp.Context(0)
    try:
        sizes = [(3, 40), (40, 900), (5, 60), (64, 2000), (64, 2000), (2, 16), (80, 3000)]
        for i, (rows, hi) in enumerate(sizes):
            step = workloads.small_step(seed=300 + i, rows=rows, n_heads=8, n_kv=2, head_dim=64, ctx_hi=hi,
                                        total_blocks=8192)
            pool = gsp.Pool.create(ctx2, total_blocks=step.total_blocks, layers=1, heads_kv=step.n_kv, head_dim=4)
            info = ctx2.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                                  step.max_seq_len)
            pool.destroy()
            print(f"case upload pack {i}: rows={rows} staging_bytes={info.staging_bytes}", flush=True)
            rows_d, ids_d, ctx_d = ctx2.download_step()
            er, ei, ec = expected_packing(step)
            assert np.array_equal(rows_d, er) and np.array_equal(ids_d, ei) and np.array_equal(ctx_d, ec), i
    finally:
        ctx2.close()
