"""Dependency inference of the task-graph backend (CPU only, RECORD_ONLY graphs).

The native runtime computes the DAG without a device in ``record`` mode; these
tests check its edges against the rules of simpler's submit path
(``runtime/pto_orchestrator.cpp:882-1254``, ``runtime/pto_dep_compute.h``):
creator edges, TensorMap overlap lookups for INPUT/INOUT, INOUT retiring a
covered writer, OUTPUT_EXISTING publishing without lookup, NO_DEP and
manual_dep skipping the map, explicit dependencies, and write-after-read
edges when a closed scope's memory is reused. The two example orchestrations
give the DAGs their reference sources imply.
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
