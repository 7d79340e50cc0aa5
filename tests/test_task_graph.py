"""Dependency inference of the task-graph backend (CPU only, RECORD_ONLY graphs).

The native runtime computes the DAG without a device in ``record`` mode; these
tests check its edges against the rules of simpler's submit path
(``runtime/pto_orchestrator.cpp:882-1254``, ``runtime/pto_dep_compute.h``):
creator edges, TensorMap overlap lookups for INPUT/INOUT, INOUT retiring a
covered writer, OUTPUT_EXISTING publishing without lookup, NO_DEP and
manual_dep skipping the map, explicit dependencies, and write-after-read
edges when a closed scope's memory is reused. The two example orchestrations
give the DAGs their reference sources imply. Seeded random programs check the
same rules as properties against an element-level model of every buffer.
"""

from __future__ import annotations

import numpy as np
import pytest

from simpler_amd.task_graph import CoreTaskArgs, IncoreKernel, TaskGraph, TaskGraphError, TensorCreateInfo
from simpler_amd.task_interface import ChipTensor, DataType

F32 = DataType.FLOAT32


def ext(addr, shape, dtype=F32):
    return ChipTensor.make(addr, shape, dtype, child_memory=True)


@pytest.fixture
def g():
    graph = TaskGraph("record")
    for fid, k in ((0, IncoreKernel.VEC_ADD), (1, IncoreKernel.VEC_ADD_SCALAR), (2, IncoreKernel.VEC_MUL)):
        graph.bind(fid, k)
    yield graph
    graph.close()


def add(g, a, b, out):
    args = CoreTaskArgs()
    args.add_input(a, b)
    args.add_output(out)
    return g.submit_task(0, args)


def copy_into(g, src, dst, tag="inout"):
    # a dependency-only task (rt_submit_dummy_task) that reads src and writes
    # dst as INOUT or OUTPUT_EXISTING: any view geometry, no kernel constraints
    args = CoreTaskArgs()
    args.add_input(src)
    if tag == "inout":
        args.add_inout(dst)
    else:
        args.add_output(dst)
    return g.rt_submit_dummy_task(args)


def test_vector_example_dag(g):
    # example_orchestration.cpp:55-112: t0 c=a+b; t1 d=c+1; t2 e=c+2; t3 g=d*e; t4 f=g+c
    a, b, f = ext(0x10000, (64,)), ext(0x20000, (64,)), ext(0x30000, (64,))
    g.orchestrate_vector_example([a, b, f])
    assert g.task_count == 5
    assert [g.fanin(i) for i in range(5)] == [[], [0], [0], [1, 2], [0, 3]]


def test_paged_attention_empty_context_gets_a_zero_fill_task():
    """An empty context has no block task; its out rows are written by one
    zero-fill task after the scope's alloc task."""
    g = TaskGraph("record")
    b, hq, d, bs, nblk, maxb = 2, 16, 64, 64, 4, 2
    lens = np.array([0, 100], np.int32)
    table = np.arange(b * maxb, dtype=np.int32).reshape(b, maxb)
    bt = ChipTensor.make(table.ctypes.data, table.shape, DataType.INT32)
    cl = ChipTensor.make(lens.ctypes.data, lens.shape, DataType.INT32)
    q = ext(0x1000000, (b, hq, d), DataType.BFLOAT16)
    kc = ext(0x2000000, (nblk, bs, 1, d), DataType.BFLOAT16)
    vc = ext(0x3000000, (nblk, bs, 1, d), DataType.BFLOAT16)
    out = ext(0x4000000, (b, hq, d))
    g.orchestrate_paged_attention([q, kc, vc, bt, cl, out], 1 / np.sqrt(d))
    # sequence 0: alloc + zero fill; sequence 1: alloc + 2 blocks x (QK, SF, PV, UP)
    assert g.task_count == 2 + (1 + 4 * 2)
    assert g.fanin(1) == []  # the fill depends on nothing
    g.close()


def test_paged_attention_dag_structure():
    g = TaskGraph("record")
    b, hq, d, bs, nblk, maxb = 2, 16, 128, 128, 16, 4
    lens = np.array([512, 300], np.int32)
    table = np.arange(b * maxb, dtype=np.int32).reshape(b, maxb)
    bt = ChipTensor.make(table.ctypes.data, table.shape, DataType.INT32)  # host tables: read by the host only
    cl = ChipTensor.make(lens.ctypes.data, lens.shape, DataType.INT32)
    q = ext(0x1000000, (b, hq, d), DataType.BFLOAT16)
    kc = ext(0x2000000, (nblk, bs, 1, d), DataType.BFLOAT16)
    vc = ext(0x3000000, (nblk, bs, 1, d), DataType.BFLOAT16)
    out = ext(0x4000000, (b, hq, d))
    g.orchestrate_paged_attention([q, kc, vc, bt, cl, out], 1 / np.sqrt(d))
    # per sequence: one alloc task + (QK, SF, PV, UP) per block (paged_attention_orch.cpp:160-248)
    assert g.task_count == (1 + 4 * 4) + (1 + 4 * 3)
    t = 0
    for seq, nb in enumerate((4, 3)):
        alloc = t
        first_seq = seq == 0
        # the second sequence's allocations reuse memory the first released:
        # those edges point back into the first sequence only
        assert g.fanin(alloc) == [] if first_seq else all(x < alloc for x in g.fanin(alloc))
        prev = None
        for bn in range(nb):
            qk, sf, pv, up = (int(x) for x in alloc + 1 + 4 * bn + np.arange(4))
            fq, fs, fp, fu = (set(g.fanin(x)) for x in (qk, sf, pv, up))
            assert sf in fp and qk in fs and {alloc, sf, pv} <= fu  # RAW chain and creator edges
            if prev is None:
                if first_seq:
                    assert fq == set() and fu == {alloc, sf, pv}
                else:
                    assert all(x < alloc for x in fq) and fu - {alloc, sf, pv} <= set(range(alloc))
            else:
                pqk, psf, ppv, pup = prev
                assert pup in fu  # INOUT chain of mi/li/oi/out over the blocks
                # the block scope closed: reused sij/pij/m/l/oi_tmp memory waits for its last readers
                assert fq == {pqk, psf} and fs == {qk, psf, ppv, pup} and fp == {sf, ppv, pup}
            prev = (qk, sf, pv, up)
        t = alloc + 1 + 4 * nb
    g.close()


def test_overlap_lookup_by_box(g):
    buf = ext(0x100000, (8, 16))
    top, bottom = buf.view((4, 16), (0, 0)), buf.view((4, 16), (4, 0))
    cols = ext(0x180000, (8, 16))
    left, right = cols.view((8, 8), (0, 0)), cols.view((8, 8), (0, 8))
    src = ext(0x200000, (4, 16))
    w = copy_into(g, src, top, "existing").task_id()  # OUTPUT_EXISTING publishes rows 0..3
    r_bottom = copy_into(g, bottom, ext(0x300000, (4, 16)), "existing").task_id()
    assert g.fanin(r_bottom) == []  # rows 4..7 do not overlap rows 0..3
    middle = buf.view((4, 16), (2, 0))
    copy_into(g, middle, ext(0x400000, (4, 16)), "existing")
    assert g.fanin(g.task_count - 1) == [w]
    # column boxes: writer of the left half, reader of the right half -> no edge
    wl = copy_into(g, ext(0x500000, (8, 8)), left, "existing").task_id()
    copy_into(g, right, ext(0x600000, (8, 8)), "existing")
    assert g.fanin(g.task_count - 1) == []
    copy_into(g, left, ext(0x700000, (8, 8)), "existing")
    assert g.fanin(g.task_count - 1) == [wl]


def test_inout_retires_covered_writer(g):
    buf = ext(0x100000, (8, 16))
    w1 = copy_into(g, ext(0x200000, (8, 16)), buf, "existing").task_id()
    w2 = copy_into(g, ext(0x300000, (8, 16)), buf, "inout").task_id()
    assert g.fanin(w2) == [w1]
    copy_into(g, buf, ext(0x400000, (8, 16)), "existing")
    assert g.fanin(g.task_count - 1) == [w2]  # w1 retired by the covering INOUT
    # a partial INOUT does not retire
    w3 = copy_into(g, ext(0x500000, (4, 16)), buf.view((4, 16), (0, 0)), "inout").task_id()
    assert g.fanin(w3) == [w2]
    copy_into(g, buf, ext(0x600000, (8, 16)), "existing")
    assert g.fanin(g.task_count - 1) == [w2, w3]


def test_output_existing_no_dep_and_manual_dep(g):
    buf = ext(0x100000, (16,))
    w1 = copy_into(g, ext(0x200000, (16,)), buf, "existing").task_id()
    w2 = copy_into(g, ext(0x300000, (16,)), buf, "existing").task_id()
    assert g.fanin(w2) == []  # OUTPUT_EXISTING does not look up earlier writers
    a = CoreTaskArgs()
    a.add_no_dep(buf)
    a.add_output(ext(0x400000, (16,)))
    a.add_scalar(1.0)
    assert g.fanin(g.submit_task(1, a).task_id()) == []  # NO_DEP: no lookup
    md = buf.view((16,), (0,), manual_dep=True)
    a = CoreTaskArgs()
    a.add_input(md)
    a.add_output(ext(0x500000, (16,)))
    a.add_scalar(1.0)
    assert g.fanin(g.submit_task(1, a).task_id()) == []  # manual_dep: creator-only
    a = CoreTaskArgs()
    a.add_input(buf)
    a.add_output(ext(0x600000, (16,)))
    a.add_scalar(1.0)
    assert g.fanin(g.submit_task(1, a).task_id()) == [w1, w2]


def test_creator_edge_and_explicit_dependencies(g):
    made = add(g, ext(0x100000, (32,)), ext(0x200000, (32,)), TensorCreateInfo((32,), F32))
    c = made.get_ref(0)
    assert c.owner_task_id == made.task_id() and c.address_space == 1 and c.buffer.addr != 0
    other = add(g, ext(0x300000, (32,)), ext(0x400000, (32,)), TensorCreateInfo((32,), F32))
    a = CoreTaskArgs()
    a.add_input(c)
    a.add_output(TensorCreateInfo((32,), F32))
    a.add_scalar(2.0)
    a.set_dependencies([other.task_id()])
    t = g.submit_task(1, a)
    assert g.fanin(t.task_id()) == [made.task_id(), other.task_id()]
    a.set_dependencies([99])
    with pytest.raises(TaskGraphError):
        g.submit_task(1, a)


def test_scope_reuse_waits_for_readers(g):
    with g.scope():
        t0 = add(g, ext(0x100000, (1024,)), ext(0x200000, (1024,)), TensorCreateInfo((1024,), F32))
        x = t0.get_ref(0)
        r1 = copy_into(g, x, ext(0x300000, (1024,)), "existing").task_id()
        r2 = copy_into(g, x, ext(0x400000, (1024,)), "existing").task_id()
    # same size: the next allocation reuses x's memory and must wait for t0, r1, r2
    t3 = add(g, ext(0x500000, (1024,)), ext(0x600000, (1024,)), TensorCreateInfo((1024,), F32))
    assert t3.get_ref(0).buffer.addr == x.buffer.addr
    assert g.fanin(t3.task_id()) == [t0.task_id(), r1, r2]
    # allocations still open are not reused
    t4 = add(g, ext(0x700000, (1024,)), ext(0x800000, (1024,)), TensorCreateInfo((1024,), F32))
    assert t4.get_ref(0).buffer.addr != t3.get_ref(0).buffer.addr and g.fanin(t4.task_id()) == []


def test_rejected_tasks_leave_no_trace(g):
    n0 = g.task_count
    a = CoreTaskArgs()
    a.add_input(ext(0x100000, (32,)), ext(0x200000, (16,)))  # sizes disagree
    a.add_output(TensorCreateInfo((32,), F32))
    with pytest.raises(TaskGraphError):
        g.submit_task(0, a)
    with pytest.raises(TaskGraphError):
        g.submit_task(7, a)  # unbound func id
    assert g.task_count == n0
    with pytest.raises(TaskGraphError):
        g.scope_end()  # no open scope
    q = TaskGraph("record")
    q.bind(0, IncoreKernel.QK_MATMUL)
    a = CoreTaskArgs()
    a.add_input(ext(0x100000, (16, 128), DataType.BFLOAT16), ext(0x200000, (64, 96), DataType.BFLOAT16))
    a.add_output(TensorCreateInfo((16, 64), F32))
    with pytest.raises(TaskGraphError):  # K mismatch: 128 vs 96
        q.submit_task(0, a)
    q.close()


def test_chip_tensor_view_matches_reference_semantics():
    t = ChipTensor.make(0x1000, (6, 10), F32)
    v = t.view((2, 4), (3, 5))
    assert v.start_offset == 3 * 10 + 5 and v.shape == (2, 4) and list(v.strides)[:2] == [10, 1]
    assert v.is_contiguous == 0 and v.extent_elem_cache == 10 + 4
    assert t.view((6, 10), (0, 0)).is_contiguous == 1
    with pytest.raises(ValueError):
        t.view((4, 4), (3, 0))


def test_register_kernel_argument_checks():
    # A record-only graph loads no code object: the checks on the arguments and
    # on each task's launch shape still apply.
    with TaskGraph("record") as g:
        for kw in (dict(block_threads=0), dict(block_threads=2048), dict(elems_per_workgroup=0),
                   dict(grid_tensor=32)):
            with pytest.raises(TaskGraphError) as e:
                g.register_kernel(5, "/nonexistent.hsaco", "k", **kw)
            assert e.value.rc == -1
        with pytest.raises(TaskGraphError):
            g.register_kernel(64, "/nonexistent.hsaco", "k")
        g.register_kernel(5, "/nonexistent.hsaco", "k", block_threads=128, grid_tensor=2, elems_per_workgroup=64)
        a, b = ext(0x10000, (4, 100)), ext(0x20000, (4, 100))
        args = CoreTaskArgs()
        args.add_input(a, b)
        with pytest.raises(TaskGraphError) as e:  # the grid follows tensor 2, the task has two
            g.submit_task(5, args)
        assert e.value.rc == -1
        assert g.task_count == 0
        args.add_output(TensorCreateInfo((4, 100), F32))
        t = g.submit_task(5, args)
        assert t.task_id() == 0 and g.fanin(0) == []
        # a registered id rebinds to a built-in and back
        g.bind(5, IncoreKernel.VEC_ADD)
        g.register_kernel(5, "/nonexistent.hsaco", "k")


def test_replay_is_graph_mode_only():
    with TaskGraph("record") as g:
        g.orchestrate_vector_example([ext(0x10000, (64,)), ext(0x20000, (64,)), ext(0x30000, (64,))])
        g.record_replay(b"key")  # nothing is kept outside GRAPH mode
        g.reset()
        assert g.replay(b"key") is False
        assert g.replay_count == 0


# ---- seeded random programs against an element-level model -----------------------------------------
#
# Each program mixes INPUT / INOUT / OUTPUT_EXISTING / OUTPUT arguments over
# views of several geometries (boxes of the buffer's own layout, flat ranges,
# strided and transposed views: the latter three are compared by byte range),
# inside nested scopes whose memory is reused. The model tracks, per element of
# every buffer, the last task that wrote it. Three properties must hold for
# every task j:
#   * every element j reads (INPUT or INOUT) was last written by an ancestor of
#     j: the creator of a runtime tensor, or the last INOUT / OUTPUT_EXISTING
#     writer of that element (an INOUT that covers and retires an older writer
#     depends on it, so the order still holds transitively);
#   * a runtime tensor placed on memory a closed scope returned has every task
#     that used the old tensor among its ancestors (write after read on reuse);
#   * every edge is justified: the target created a tensor j passes, wrote a
#     byte range j reads or updates, or used the memory j's new tensor reuses.

def _elements(t: ChipTensor) -> np.ndarray:
    idx = np.array([int(t.start_offset)], dtype=np.int64)
    for d in range(int(t.ndims)):
        step = np.arange(int(t.shapes[d]), dtype=np.int64) * int(t.strides[d])
        idx = (idx[:, None] + step[None, :]).ravel()
    return idx


def _byte_range(t: ChipTensor) -> tuple[int, int]:
    last = sum((int(t.shapes[d]) - 1) * int(t.strides[d]) for d in range(int(t.ndims)))
    return 4 * int(t.start_offset), 4 * (int(t.start_offset) + last + 1)


def _random_view(rng, base: ChipTensor, external: bool) -> ChipTensor:
    rows, cols = base.shape
    kind = int(rng.integers(0, 5 if external else 2))
    if kind == 0:
        return base
    if kind == 1:  # a box of the buffer's own layout
        h, w = int(rng.integers(1, rows + 1)), int(rng.integers(1, cols + 1))
        return base.view((h, w), (int(rng.integers(0, rows - h + 1)), int(rng.integers(0, cols - w + 1))))
    addr, n = base.buffer.addr, rows * cols
    if kind == 2:  # a flat range (dense, another geometry)
        k = int(rng.integers(1, n + 1))
        return ext(addr, (n,)).view((k,), (int(rng.integers(0, n - k + 1)),))
    if kind == 3:  # every other element (not dense)
        k = int(rng.integers(1, n // 2 + 1))
        return ChipTensor.make(addr, (n // 2,), F32, True, strides=(2,)).view((k,), (int(rng.integers(0, n // 2 - k + 1)),))
    w, h = int(rng.integers(1, cols + 1)), int(rng.integers(1, rows + 1))  # transposed
    t = ChipTensor.make(addr, (cols, rows), F32, True, strides=(1, cols))
    return t.view((w, h), (int(rng.integers(0, cols - w + 1)), int(rng.integers(0, rows - h + 1))))


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_random_programs_keep_every_read_after_its_writer(seed):
    rng = np.random.default_rng(seed)
    g = TaskGraph("record")
    externals = [ext(0x1000000 * (i + 1), (8, 16)) for i in range(3)]
    last = {t.buffer.addr: np.full(8 * 16, -1, dtype=np.int64) for t in externals}  # addr -> last writer
    hist = {t.buffer.addr: [] for t in externals}  # addr -> [(task, byte range)] of published writes
    live = {t.buffer.addr: t for t in externals}  # tensors a task may pass
    users: dict[int, set[int]] = {}  # runtime tensor addr -> tasks that passed it
    span: dict[int, tuple[int, int]] = {}  # runtime tensor addr -> absolute byte range
    scopes: list[list[int]] = []
    freed: list[tuple[int, int, set[int]]] = []
    anc: list[int] = []  # ancestor bitsets
    shapes = [(8, 16), (4, 16), (3, 16), (16, 16)]
    for j in range(400):
        if rng.random() < 0.08 and len(scopes) < 3:
            g.scope_begin()
            scopes.append([])
        if rng.random() < 0.06 and scopes:
            g.scope_end()
            for addr in scopes.pop():
                freed.append((*span.pop(addr), users.pop(addr)))
                del live[addr], last[addr], hist[addr]
        args, roles = CoreTaskArgs(), []
        pool = list(live.values())
        for _ in range(int(rng.integers(0, 3))):
            base = pool[int(rng.integers(0, len(pool)))]
            v = _random_view(rng, base, base.buffer.addr not in users)
            args.add_input(v)
            roles.append(("in", v))
        for role in ("inout", "existing"):
            if rng.random() < 0.4:
                base = pool[int(rng.integers(0, len(pool)))]
                v = _random_view(rng, base, base.buffer.addr not in users)
                (args.add_inout if role == "inout" else args.add_output)(v)
                roles.append((role, v))
        if not roles or rng.random() < 0.35:
            args.add_output(TensorCreateInfo(shapes[int(rng.integers(0, len(shapes)))], F32))
            roles.append(("create", None))
        made = g.rt_submit_dummy_task(args)
        assert made.task_id() == j
        fanin = g.fanin(j)
        assert all(0 <= i < j for i in fanin), (j, fanin)
        a = 0
        for i in fanin:
            a |= anc[i] | (1 << i)
        anc.append(a)

        justified = set()
        for role, v in roles:
            if role == "create":
                continue
            addr = v.buffer.addr
            if v.owner_task_id != 0xFFFFFFFFFFFFFFFF:
                justified.add(int(v.owner_task_id))
            if role in ("in", "inout"):
                for w in set(last[addr][_elements(v)].tolist()) - {-1}:
                    assert a >> w & 1, f"seed {seed}: task {j} reads what task {w} wrote; fanin {fanin}"
                b, e = _byte_range(v)
                justified.update(w for w, (wb, we) in hist[addr] if wb < e and b < we)
        created = iter(made.get_ref(i) for i in range(made.size()))
        for role, v in roles:
            if role != "create":
                continue
            t = next(created)
            b, e = t.buffer.addr, t.buffer.addr + 4 * int(np.prod(t.shape))
            for fb, fe, who in [f for f in freed if f[0] < e and b < f[1]]:
                for u in who:
                    assert a >> u & 1, f"seed {seed}: task {j} reuses memory task {u} used; fanin {fanin}"
                justified.update(who)
                freed.remove((fb, fe, who))
            live[b], last[b], hist[b], users[b], span[b] = t, np.full(int(np.prod(t.shape)), j), [], {j}, (b, e)
            if scopes:
                scopes[-1].append(b)
        assert set(fanin) <= justified, f"seed {seed}: task {j} has unjustified edges {set(fanin) - justified}"
        for role, v in roles:
            if role == "create":
                continue
            addr = v.buffer.addr
            if addr in users:
                users[addr].add(j)
            if role in ("inout", "existing"):
                last[addr][_elements(v)] = j
                hist[addr].append((j, _byte_range(v)))
    g.close()
