"""Seeded random programs on the task-graph backend, EAGER and GRAPH, against numpy.

Each program submits 150 tasks of the built-in vector kernels (add, add scalar,
mul) and zero fills. Their operands are row ranges and flat ranges of three
device buffers, and row ranges of runtime tensors created inside nested scopes
whose memory is reused. Outputs are new tensors, existing views disjoint from
the task's inputs, or in place (INOUT on one of the inputs). Programs also
read runtime tensors part way through (a read drains the pending work) and
close GRAPH segments at random points; a seed gives the same program in both
modes.

The kernels are fp32 element-wise operations, so every value is bit-exact
against the same operation in numpy. Each program runs twice on a reset graph,
with new external values at the same addresses: in GRAPH mode the second run
relaunches the cached executable graphs, which must read the new values.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from simpler_amd.task_graph import CoreTaskArgs, IncoreKernel, TaskGraph, TensorCreateInfo
from simpler_amd.task_interface import ChipTensor, DataType

pytestmark = pytest.mark.gpu

F32 = DataType.FLOAT32
W = 64  # row width of every buffer
ROWS = 8  # rows of each external buffer
ADD, ADD_SCALAR, MUL, ZERO = 0, 1, 2, 3


def _span(v: ChipTensor) -> tuple[int, int]:
    """[first, last] + 1 element of a view in its buffer."""
    last = sum((int(v.shapes[d]) - 1) * int(v.strides[d]) for d in range(int(v.ndims)))
    return int(v.start_offset), int(v.start_offset) + last + 1


def _elements(v: ChipTensor) -> np.ndarray:
    idx = np.array([int(v.start_offset)], dtype=np.int64)
    for d in range(int(v.ndims)):
        idx = (idx[:, None] + np.arange(int(v.shapes[d]), dtype=np.int64)[None, :] * int(v.strides[d])).ravel()
    return idx


def _disjoint(a: ChipTensor, b: ChipTensor) -> bool:
    if a.buffer.addr != b.buffer.addr:
        return True
    (ab, ae), (bb, be) = _span(a), _span(b)
    return ae <= bb or be <= ab


def run_program(g: TaskGraph, externals: list[torch.Tensor], seed: int, mode: str) -> int:
    """Submits the seed's program, checks every read, returns the number of values checked."""
    rng = np.random.default_rng(seed)
    model: dict[int, np.ndarray] = {}  # buffer address -> its values, flat
    live: dict[int, ChipTensor] = {}  # buffer address -> a 2-D [rows, W] tensor over it
    runtime: set[int] = set()
    for x in externals:
        t = ChipTensor.make(x.data_ptr(), (ROWS, W), F32, child_memory=True)
        model[t.buffer.addr] = x.cpu().numpy().reshape(-1).copy()
        live[t.buffer.addr] = t
    scopes: list[list[int]] = []
    checked = 0

    def pick(h: int) -> ChipTensor:
        cands = [t for t in live.values() if t.shape[0] >= h]
        base = cands[int(rng.integers(0, len(cands)))]
        if base.buffer.addr not in runtime and rng.random() < 0.4:  # a flat range at any offset
            total = ROWS * W
            flat = ChipTensor.make(base.buffer.addr, (total,), F32, child_memory=True)
            return flat.view((h * W,), (int(rng.integers(0, total - h * W + 1)),))
        return base.view((h, W), (int(rng.integers(0, base.shape[0] - h + 1)), 0))

    def read_and_check(t: ChipTensor) -> int:
        got = g.read(t).reshape(-1)
        np.testing.assert_array_equal(got, model[t.buffer.addr][_elements(t)], err_msg=f"seed {seed} {mode}")
        return got.size

    for j in range(150):
        if rng.random() < 0.08 and len(scopes) < 3:
            g.scope_begin()
            scopes.append([])
        if rng.random() < 0.06 and scopes:
            g.scope_end()
            for addr in scopes.pop():
                del live[addr], model[addr]
                runtime.discard(addr)
        op = int(rng.integers(0, 4))
        h = int(rng.choice([1, 2, 3, 4, 8]))
        args = CoreTaskArgs()
        if op == ZERO:
            base = [t for t in live.values() if t.shape[0] >= h]
            base = base[int(rng.integers(0, len(base)))]
            w = int(rng.integers(1, W + 1))
            dst = base.view((h, w), (int(rng.integers(0, base.shape[0] - h + 1)), int(rng.integers(0, W - w + 1))))
            kind = ("create", "existing", "inout")[int(rng.integers(0, 3))]
            if kind == "create":
                dst = None
                args.add_output(TensorCreateInfo((h, W), F32))
            elif kind == "existing":
                args.add_output(dst)
            else:
                args.add_inout(dst)
            result = np.zeros(h * (W if dst is None else w), dtype=np.float32)
            made = g.submit_task(ZERO, args)
        else:
            ins = [pick(h) for _ in range(1 if op == ADD_SCALAR else 2)]
            vals = [model[v.buffer.addr][_elements(v)] for v in ins]
            if op == ADD:
                result = vals[0] + vals[1]
            elif op == MUL:
                result = vals[0] * vals[1]
            else:
                s = np.float32(rng.standard_normal())
                result = vals[0] + s
            args.add_input(*ins)
            kind = ("create", "existing", "inout")[int(rng.integers(0, 3))]
            dst = None
            if kind == "inout":  # in place on one of the inputs
                dst = ins[int(rng.integers(0, len(ins)))]
                args.add_inout(dst)
            elif kind == "existing":
                for _ in range(10):
                    cand = pick(h)
                    if all(_disjoint(cand, v) for v in ins):
                        dst = cand
                        break
                if dst is None:
                    kind = "create"
                else:
                    args.add_output(dst)
            if kind == "create":
                args.add_output(TensorCreateInfo((h, W), F32))
            if op == ADD_SCALAR:
                args.add_scalar(float(s))
            made = g.submit_task(op, args)
        if dst is None:
            t = made.get_ref(0)
            addr = t.buffer.addr
            assert addr not in live, f"seed {seed}: task {j} got the memory of a live tensor"
            live[addr], model[addr] = t, result.copy()
            runtime.add(addr)
            if scopes:
                scopes[-1].append(addr)
        else:
            model[dst.buffer.addr][_elements(dst)] = result
        if rng.random() < 0.05 and runtime:
            addr = sorted(runtime)[int(rng.integers(0, len(runtime)))]
            checked += read_and_check(live[addr])
        if rng.random() < 0.05:  # closes a GRAPH segment; EAGER has launched everything already
            g.launch()
    g.launch()
    g.wait()
    for x in externals:
        addr = x.data_ptr()
        np.testing.assert_array_equal(x.cpu().numpy().reshape(-1), model[addr], err_msg=f"seed {seed} {mode}")
        checked += model[addr].size
    for addr in sorted(runtime):
        checked += read_and_check(live[addr])
    return checked


@pytest.mark.parametrize("mode", ["eager", "graph"])
@pytest.mark.parametrize("seed", [31, 32, 33])
def test_random_programs_match_numpy(device, seed, mode):
    print(f"[case] tg random program seed={seed} mode={mode}", flush=True)
    data = np.random.default_rng(seed + 1000)
    externals = [torch.zeros((ROWS, W), dtype=torch.float32, device=device) for _ in range(3)]
    with TaskGraph(mode) as g:
        for fid, k in ((ADD, IncoreKernel.VEC_ADD), (ADD_SCALAR, IncoreKernel.VEC_ADD_SCALAR),
                       (MUL, IncoreKernel.VEC_MUL), (ZERO, IncoreKernel.ZERO_FILL)):
            g.bind(fid, k)
        for run in range(2):
            g.reset()
            for x in externals:  # new values at the same addresses
                x.copy_(torch.from_numpy(data.standard_normal((ROWS, W)).astype(np.float32)))
            torch.cuda.synchronize(device)
            checked = run_program(g, externals, seed, mode)
            assert checked > 3 * ROWS * W, f"run {run}"
