"""GPU parity of the task-graph backend: incore kernels, orchestrations, hipGraph replays.

* Each incore kernel against the oracle's step function (``oracle.pa_oracle``
  qk_matmul / softmax_prepare / pv_matmul / online_update, pinned in
  test_task_graph_oracle.py). Matmuls: fp32 sums in another order, so
  |diff| <= 1e-4 + 1e-5·|x|. Softmax: m exact; p on the bf16 grid and at most one
  bf16 step from the oracle (device and host exp may differ in the last fp32
  bit before rounding); l within 1e-5 relative. Online update: exp as above,
  within 1e-5 relative.
* The reference paged-attention orchestration (QK -> SF -> PV -> UP per block)
  end to end, eager and as a hipGraph, through the TaskGraph API and through
  simpler_run (Worker execution="eager"/"graph"), against the whole-op oracle
  at the decode tolerance (max-abs 2e-2, rel-L2 1e-3).
* The vector example: f = (a+b+1)*(a+b+2) + (a+b) is fp32 arithmetic in a fixed
  order, so it is bit-exact against numpy in the same order (and 47.0 for the
  reference's a = 2, b = 3).
* hipGraph execution replays the same instantiated graph; every replay is
  checked against the eager result, with the program's own eager work and
  synchronisations in between.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import pa_oracle as po
from simpler_amd import TaskArgs, Worker
from simpler_amd import paged_attention as pa
from simpler_amd.task_graph import CoreTaskArgs, IncoreKernel, TaskGraph, TaskGraphError, TensorCreateInfo
from simpler_amd.task_graph import vector_example_callable
from simpler_amd.task_interface import ChipTensor, DataType, TensorArgType
from simpler_amd.workloads import make_case, make_custom_case
from tests.pa_helpers import assert_close, oracle_numpy

pytestmark = pytest.mark.gpu

_DT = {torch.bfloat16: DataType.BFLOAT16, torch.float32: DataType.FLOAT32, torch.int32: DataType.INT32}


def ct(t: torch.Tensor) -> ChipTensor:
    assert t.is_contiguous()
    return ChipTensor.make(t.data_ptr(), tuple(t.shape), _DT[t.dtype], child_memory=t.device.type != "cpu")


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def bf16_dev(rng, shape, device, scale=1.0):
    x = torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32))
    return x.to(torch.bfloat16).to(device)


@pytest.fixture
def graph(device):
    g = TaskGraph("eager")
    for k in (IncoreKernel.QK_MATMUL, IncoreKernel.SOFTMAX_PREPARE, IncoreKernel.PV_MATMUL,
              IncoreKernel.ONLINE_UPDATE):
        g.bind(int(k), k)
    yield g
    g.close()


def close_matmul(got, want):
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-5 * np.abs(want)), np.abs(got - want).max()


@pytest.mark.parametrize("m,n,d", [(16, 128, 128), (64, 64, 64), (20, 48, 96)])
def test_qk_and_pv_kernels(graph, device, m, n, d):
    print(f"[case] tg qk/pv m={m} n={n} d={d}", flush=True)
    rng = np.random.default_rng(m * 7 + n)
    q = bf16_dev(rng, (m, d), device)
    cache = bf16_dev(rng, (4 * n, d), device)  # kj is a view at block 2
    kj = ct(cache).view((n, d), (2 * n, 0))
    a = CoreTaskArgs()
    a.add_input(ct(q), kj)
    a.add_output(TensorCreateInfo((m, n), DataType.FLOAT32))
    sij = graph.submit_task(0, a).get_ref(0)
    got_s = graph.read(sij)
    close_matmul(got_s, po.qk_matmul(to_np(q), to_np(cache)[2 * n: 3 * n]))

    p = torch.from_numpy(po.bf16_round(np.abs(rng.standard_normal((m, n))).astype(np.float32))).to(torch.bfloat16)
    p = p.to(device)
    v = bf16_dev(rng, (4 * n, d), device)
    a = CoreTaskArgs()
    a.add_input(ct(p), ct(v).view((n, d), (n, 0)))
    a.add_output(TensorCreateInfo((m, d), DataType.FLOAT32))
    o = graph.submit_task(2, a).get_ref(0)
    close_matmul(graph.read(o), po.pv_matmul(to_np(p), to_np(v)[n: 2 * n]))


@pytest.mark.parametrize("valid", [1, 57, 128, 0])
def test_softmax_prepare_kernel(graph, device, valid):
    print(f"[case] tg softmax valid={valid}", flush=True)
    rng = np.random.default_rng(100 + valid)
    m, n = 16, 128
    s = torch.from_numpy((rng.standard_normal((m, n)) * 6).astype(np.float32)).to(device)
    scale = 0.0883883
    a = CoreTaskArgs()
    a.add_input(ct(s).view((m, valid), (0, 0)) if valid else ct(s).view((m, 0), (0, 0)))
    a.add_output(TensorCreateInfo((m, n), DataType.BFLOAT16), TensorCreateInfo((m,), DataType.FLOAT32),
                 TensorCreateInfo((m,), DataType.FLOAT32))
    a.add_scalar(ctypes.c_float(scale))
    outs = graph.submit_task(1, a)
    p = graph.read(outs.get_ref(0))
    mm, ll = graph.read(outs.get_ref(1)), graph.read(outs.get_ref(2))
    wp, wm, wl = po.softmax_prepare(to_np(s), valid, scale)
    np.testing.assert_array_equal(mm, wm)
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(wp), 1e-30))) - 7)
    assert np.all(np.abs(p - wp) <= step * 1.0001)
    assert np.array_equal(p, po.bf16_round(p))
    np.testing.assert_allclose(ll, wl, rtol=1e-5, atol=1e-6)


def test_online_update_kernel_chain(graph, device):
    print("[case] tg online_update chain", flush=True)
    rng = np.random.default_rng(7)
    m, d = 16, 128
    blocks = [(rng.standard_normal(m).astype(np.float32) * 3, (rng.random(m) * 50 + 1).astype(np.float32),
               rng.standard_normal((m, d)).astype(np.float32) * 10) for _ in range(3)]
    state = graph.alloc_tensors(TensorCreateInfo((m, d), DataType.FLOAT32), TensorCreateInfo((m,), DataType.FLOAT32),
                                TensorCreateInfo((m,), DataType.FLOAT32))
    oi, li, mi = state.get_ref(0), state.get_ref(1), state.get_ref(2)
    dst = torch.zeros((m, d), dtype=torch.float32, device=device)
    keep = []
    wm = wl = wo = None
    for k, (mb, lb, ob) in enumerate(blocks):
        tens = [torch.from_numpy(x).to(device) for x in (mb, lb, ob)]
        keep += tens
        a = CoreTaskArgs()
        a.add_input(*(ct(t) for t in tens))
        a.add_inout(mi, li, oi, ct(dst))
        a.add_scalar(int(k == 0), int(k == len(blocks) - 1))
        graph.submit_task(3, a)
        wm, wl, wo, wd = po.online_update(mb, lb, ob, wm, wl, wo, k == 0, k == len(blocks) - 1)
    torch.cuda.synchronize(device)
    np.testing.assert_array_equal(graph.read(mi), wm)
    np.testing.assert_allclose(graph.read(li), wl, rtol=1e-5)
    np.testing.assert_allclose(dst.cpu().numpy(), wd, rtol=1e-5, atol=1e-6)


def _pa_tensors(case, d):
    return [ct(d.query), ct(d.key_cache), ct(d.value_cache), ct(d.block_table), ct(d.context_lens)]


@pytest.mark.parametrize("mode", ["eager", "graph"])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_paged_attention_orchestration(device, mode, out_dtype):
    print(f"[case] tg paged attention mode={mode} out={out_dtype}", flush=True)
    case = make_case("cfg1_small")
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=out_dtype, device=device)
    with TaskGraph(mode) as g:
        g.orchestrate_paged_attention(_pa_tensors(case, d) + [ct(out)], case.scale)
        assert g.task_count == 2 * (1 + 4 * 4)
        g.launch()
        g.wait()
    ref = oracle_numpy(case)
    if out_dtype == torch.bfloat16:
        ref = torch.tensor(ref).to(torch.bfloat16).float().numpy()
    assert_close(out.float().cpu().numpy(), ref, what=f"task graph {mode}")


def test_paged_attention_ragged_and_multi_tile(device):
    # 256 heads -> two 128-row q tiles per sequence (paged_attention_orch.cpp:105-106); ragged lengths
    print("[case] tg paged attention ragged 256 heads", flush=True)
    case = make_custom_case(batch=3, num_heads=256, kv_heads=1, head_dim=64, block_size=64,
                            context_lens=[1, 65, 200], seed=5, max_blocks=4)
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    with TaskGraph("eager") as g:
        g.orchestrate_paged_attention(_pa_tensors(case, d) + [ct(out)], case.scale)
        g.wait()
    assert_close(out.cpu().numpy(), oracle_numpy(case), what="task graph ragged")


@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_empty_context_writes_zeros(device, mode):
    """An empty context submits no block task; the orchestration writes its rows
    as zeros (a zero-fill task), as the fused decode defines them."""
    print(f"[case] tg empty context mode={mode}", flush=True)
    case = make_custom_case(batch=3, num_heads=16, kv_heads=1, head_dim=64, block_size=64,
                            context_lens=[0, 65, 0], seed=6, max_blocks=2)
    d = case.to(device)
    out = torch.full(case.out_shape(), float("nan"), dtype=torch.float32, device=device)
    with TaskGraph(mode) as g:
        g.orchestrate_paged_attention(_pa_tensors(case, d) + [ct(out)], case.scale)
        g.launch()
        g.wait()
    got = out.cpu().numpy()
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert_close(got, oracle_numpy(case), what=f"task graph empty context {mode}")


def test_bad_block_is_reported_before_any_launch(device):
    case = make_case("cfg1_small")
    d = case.to(device)
    bt = d.block_table.clone()
    bt[1, 2] = case.key_cache.shape[0] + 3
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    with TaskGraph("graph") as g:
        with pytest.raises(TaskGraphError) as e:
            g.orchestrate_paged_attention([ct(d.query), ct(d.key_cache), ct(d.value_cache), ct(bt),
                                           ct(d.context_lens), ct(out)], case.scale)
        assert e.value.rc == -6  # SIMPLER_HIP_ERR_BAD_BLOCK


def test_hipgraph_replays_match_eager(device):
    print("[case] tg hipGraph replays", flush=True)
    case = make_custom_case(batch=2, num_heads=16, kv_heads=1, head_dim=128, block_size=128,
                            context_lens=[300, 512], seed=9, max_blocks=4)
    d = case.to(device)
    eager_out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    with TaskGraph("eager") as g:
        g.orchestrate_paged_attention(_pa_tensors(case, d) + [ct(eager_out)], case.scale)
        g.wait()
    want = eager_out.cpu().numpy()
    # a second query/out pair: replays alternate between them, so the cached
    # graph's kernel parameters are patched in place every other run
    q2 = (d.query.float() * -0.5).to(torch.bfloat16).contiguous()
    eager2 = torch.zeros_like(eager_out)
    with TaskGraph("eager") as g:
        g.orchestrate_paged_attention([ct(q2)] + _pa_tensors(case, d)[1:] + [ct(eager2)], case.scale)
        g.wait()
    want2 = eager2.cpu().numpy()
    out, out2 = torch.zeros_like(eager_out), torch.zeros_like(eager_out)
    with TaskGraph("graph") as g:
        for rep in range(6):
            g.reset()
            alt = rep % 2 == 1
            tensors = ([ct(q2)] + _pa_tensors(case, d)[1:] + [ct(out2)]) if alt else (_pa_tensors(case, d) + [ct(out)])
            g.orchestrate_paged_attention(tensors, case.scale)
            g.launch()
            g.wait()
            got = (out2 if alt else out).cpu().numpy()
            np.testing.assert_array_equal(got, want2 if alt else want, err_msg=f"replay {rep}")
            (out2 if alt else out).fill_(float("nan"))  # eager work between replays
            torch.cuda.synchronize(device)


def test_vector_example_through_graph_api(device):
    rng = np.random.default_rng(3)
    a = torch.from_numpy(rng.standard_normal(128 * 128).astype(np.float32)).to(device)
    b = torch.from_numpy(rng.standard_normal(128 * 128).astype(np.float32)).to(device)
    f = torch.zeros_like(a)
    for mode in ("eager", "graph"):
        f.zero_()
        with TaskGraph(mode) as g:
            g.scope_begin()
            g.orchestrate_vector_example([ct(a), ct(b), ct(f)])
            g.scope_end()
            g.launch()
            g.wait()
        an, bn = a.cpu().numpy(), b.cpu().numpy()
        c = an + bn
        np.testing.assert_array_equal(f.cpu().numpy(), (c + np.float32(1)) * (c + np.float32(2)) + c)


@pytest.mark.parametrize("execution", ["eager", "graph"])
def test_worker_runs_reference_chain_on_the_task_graph(device, execution):
    print(f"[case] worker execution={execution}", flush=True)
    w = Worker(level=2, platform="mi355x", device_id=device.index or 0, execution=execution)
    w.init()
    try:
        case = make_custom_case(batch=4, num_heads=16, kv_heads=1, head_dim=16, block_size=16,
                                context_lens=[33, 64, 128, 15], seed=42, max_blocks=16)  # CaseVarSeq4
        h = w.register(pa.reference_chain_callable())
        out = torch.zeros(case.out_shape(), dtype=torch.float32)
        args = TaskArgs()
        for t in (case.query, case.key_cache, case.value_cache, case.block_table, case.context_lens):
            args.add_tensor(t.contiguous(), TensorArgType.INPUT)
        args.add_tensor(out, TensorArgType.OUTPUT_EXISTING)
        args.add_scalar(ctypes.c_float(case.scale))
        for _ in range(2):  # second run reuses the context's graph (hipGraph: updated in place)
            out.zero_()
            w.run(h, args)
            assert_close(out.numpy(), oracle_numpy(case), what=f"worker {execution}")
        # the vector example callable (reference golden: a=2, b=3 -> f=47)
        hv = w.register(vector_example_callable())
        va = TaskArgs()
        a, b, f = torch.full((128 * 128,), 2.0), torch.full((128 * 128,), 3.0), torch.zeros(128 * 128)
        va.add_tensor(a, TensorArgType.INPUT)  # TaskArgs keeps addresses only: a, b, f stay referenced here
        va.add_tensor(b, TensorArgType.INPUT)
        va.add_tensor(f, TensorArgType.OUTPUT_EXISTING)
        w.run(hv, va)
        assert torch.all(f == 47.0)
    finally:
        w.close()


# ---- kernels of the caller's own (simpler_hip_tg_register_kernel) -----------------------------------

_CODE_OBJECT = Path(__file__).resolve().parent / "kernels" / "_build" / "tg_user_kernels.hsaco"


@pytest.fixture(scope="module")
def user_code_object():
    if not _CODE_OBJECT.exists():  # built by __graft_entry__.build(); build it here only if missing
        from simpler_amd import build as native_build
        native_build.build_code_object(_CODE_OBJECT.parent.parent / "tg_user_kernels.hip", _CODE_OBJECT)
    return _CODE_OBJECT


@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_registered_kernels_run_a_dag(device, user_code_object, mode):
    # y0 = alpha*x + b (registered), y1 = y0 * s[row] into rows 4..11 of an
    # external tensor (registered, a view with an offset), y2 = y1 + x (built-in)
    print(f"[case] tg registered kernels mode={mode}", flush=True)
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((8, 96)).astype(np.float32)).to(device)
    b = torch.from_numpy(rng.standard_normal((8, 96)).astype(np.float32)).to(device)
    s = torch.from_numpy(rng.standard_normal(8).astype(np.float32)).to(device)
    big = torch.full((16, 96), float("nan"), dtype=torch.float32, device=device)
    big_ct = ct(big)
    rows = big_ct.view([8, 96], [4, 0])
    xn, bn, sn = x.cpu().numpy(), b.cpu().numpy(), s.cpu().numpy()
    with TaskGraph(mode) as g:
        g.register_kernel(10, user_code_object, "tg_axpb", block_threads=256, grid_tensor=2, elems_per_workgroup=256)
        g.register_kernel(11, user_code_object, "tg_row_scale", block_threads=128, grid_tensor=-1,
                          elems_per_workgroup=3)
        g.bind(12, IncoreKernel.VEC_ADD)
        for rep, alpha in enumerate((1.5, -0.25, 1.5)):
            g.reset()
            a0 = CoreTaskArgs()
            a0.add_input(ct(x), ct(b))
            a0.add_output(TensorCreateInfo((8, 96), DataType.FLOAT32))
            a0.add_scalar(float(alpha))
            y0 = g.submit_task(10, a0).get_ref(0)
            a1 = CoreTaskArgs()
            a1.add_input(y0, ct(s))
            a1.add_output(rows)  # OUTPUT_EXISTING: a view of the external tensor
            t1 = g.submit_task(11, a1)
            a2 = CoreTaskArgs()
            a2.add_input(rows, ct(x))
            a2.add_output(TensorCreateInfo((8, 96), DataType.FLOAT32))
            t2 = g.submit_task(12, a2)
            assert g.fanin(t1.task_id()) == [0] and g.fanin(t2.task_id()) == [1]
            g.launch()
            y2 = g.read(t2.get_ref(0))
            g.wait()
            want1 = (np.float32(alpha) * xn + bn) * sn[:, None]
            np.testing.assert_allclose(big[4:12].cpu().numpy(), want1, rtol=1e-6, atol=1e-6, err_msg=f"rep {rep}")
            np.testing.assert_allclose(y2.reshape(8, 96), want1 + xn, rtol=1e-6, atol=1e-6, err_msg=f"rep {rep}")
            assert torch.isnan(big[:4]).all() and torch.isnan(big[12:]).all()  # nothing outside the view
            big.fill_(float("nan"))  # eager work between the runs
            torch.cuda.synchronize(device)


def test_registered_kernel_that_cannot_load_is_refused(device, user_code_object, tmp_path):
    with TaskGraph("eager") as g:
        with pytest.raises(TaskGraphError) as e:
            g.register_kernel(3, tmp_path / "missing.hsaco", "tg_axpb")
        assert e.value.rc == -2
        with pytest.raises(TaskGraphError) as e:
            g.register_kernel(3, user_code_object, "no_such_kernel")
        assert e.value.rc == -2


# ---- whole-step replay (GRAPH mode) --------------------------------------------------------------------

def test_orchestration_step_replays_until_its_tables_change(device):
    print("[case] tg paged attention step replay", flush=True)
    case = make_case("cfg1_small")
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    tensors = _pa_tensors(case, d) + [ct(out)]
    q0 = d.query.clone()
    with TaskGraph("graph") as g:
        def step(expect_replays):
            g.reset()
            out.fill_(float("nan"))
            torch.cuda.synchronize(device)
            g.orchestrate_paged_attention(tensors, case.scale)
            assert g.replay_count == expect_replays
            g.launch()
            g.wait()
            return out.cpu().numpy()

        assert_close(step(0), oracle_numpy(case), what="first step")
        assert_close(step(1), oracle_numpy(case), what="replayed step")
        assert g.task_count == 2 * (1 + 4 * 4)
        # new query values at the same address: the key holds; the graph reads them
        d.query.copy_((q0.float() * -0.75).to(torch.bfloat16))
        case.query = d.query.cpu()
        assert_close(step(2), oracle_numpy(case), what="replay, new query values")
        # a shorter context: the tables changed, so the step is orchestrated again
        d.context_lens[1] = 300
        case.context_lens = d.context_lens.cpu()
        assert_close(step(2), oracle_numpy(case), what="new tables")
        assert g.task_count == 2 + 4 * 4 + 4 * 3
        assert_close(step(3), oracle_numpy(case), what="replay of the new tables")


def test_eager_graphs_do_not_replay(device):
    case = make_case("cfg1_small")
    d = case.to(device)
    out = torch.zeros(case.out_shape(), dtype=torch.float32, device=device)
    with TaskGraph("eager") as g:
        for _ in range(2):
            g.reset()
            g.orchestrate_paged_attention(_pa_tensors(case, d) + [ct(out)], case.scale)
            g.wait()
        assert g.replay_count == 0
    assert_close(out.cpu().numpy(), oracle_numpy(case), what="eager")


def test_user_step_with_registered_kernels_replays(device, user_code_object):
    # A caller's own step (two registered kernels and a built-in) recorded under
    # a key, then replayed on reset graphs: new input values at the same
    # addresses flow through; a different key orchestrates again.
    print("[case] tg user step record/replay", flush=True)
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.standard_normal((4, 64)).astype(np.float32)).to(device)
    b = torch.from_numpy(rng.standard_normal((4, 64)).astype(np.float32)).to(device)
    s = torch.from_numpy(rng.standard_normal(4).astype(np.float32)).to(device)
    out = torch.zeros((4, 64), dtype=torch.float32, device=device)
    with TaskGraph("graph") as g:
        g.register_kernel(10, user_code_object, "tg_axpb", block_threads=256, grid_tensor=2, elems_per_workgroup=256)
        g.register_kernel(11, user_code_object, "tg_row_scale", block_threads=128, grid_tensor=2,
                          elems_per_workgroup=128)
        g.bind(12, IncoreKernel.VEC_ADD)

        def step(alpha: float) -> None:
            key = f"axpb-rowscale-add alpha={alpha}".encode()
            g.reset()
            if not g.replay(key):
                a0 = CoreTaskArgs()
                a0.add_input(ct(x), ct(b))
                a0.add_output(TensorCreateInfo((4, 64), DataType.FLOAT32))
                a0.add_scalar(float(alpha))
                y0 = g.submit_task(10, a0).get_ref(0)
                a1 = CoreTaskArgs()
                a1.add_input(y0, ct(s))
                a1.add_output(TensorCreateInfo((4, 64), DataType.FLOAT32))
                y1 = g.submit_task(11, a1).get_ref(0)
                a2 = CoreTaskArgs()
                a2.add_input(y1, ct(x))
                a2.add_output(ct(out))
                g.submit_task(12, a2)
                g.record_replay(key)
            g.launch()
            g.wait()

        def want(alpha: float) -> np.ndarray:
            xn, bn, sn = x.cpu().numpy(), b.cpu().numpy(), s.cpu().numpy()
            return (np.float32(alpha) * xn + bn) * sn[:, None] + xn

        step(2.0)
        np.testing.assert_allclose(out.cpu().numpy(), want(2.0), rtol=1e-6, atol=1e-6)
        assert g.replay_count == 0
        x.mul_(-1.5)  # new values, same address: the recorded step still applies
        out.fill_(float("nan"))
        step(2.0)
        assert g.replay_count == 1 and g.task_count == 3
        np.testing.assert_allclose(out.cpu().numpy(), want(2.0), rtol=1e-6, atol=1e-6)
        step(0.5)  # another key: orchestrated and recorded again
        assert g.replay_count == 1
        np.testing.assert_allclose(out.cpu().numpy(), want(0.5), rtol=1e-6, atol=1e-6)
        step(0.5)
        assert g.replay_count == 2
        np.testing.assert_allclose(out.cpu().numpy(), want(0.5), rtol=1e-6, atol=1e-6)
