"""The operator boundary as the reference's callers use it: ``aligned_gather_cat4`` in its
six-argument form, the engine's ``OpDispatcher`` entry points, the builders' reference
defaults, and the reference-side ctypes binding of the integration guide run as written."""
import inspect
import os
import re

import numpy as np
import pytest

from oracle import nl as onl
from oracle import ops as oops
from fastmd_amd import systems

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _params(fn):
    return list(inspect.signature(fn).parameters.values())


def test_aligned_gather_cat4_takes_the_reference_arguments():
    from fastmd_amd.ops.gather_cat import aligned_gather_cat3, aligned_gather_cat4

    # triton_gather_cat.py:181-186 and :353-360
    assert [p.name for p in _params(aligned_gather_cat3)] == ["aligned", "gathered", "index_a", "index_b"]
    assert [p.name for p in _params(aligned_gather_cat4)] == ["aligned", "gathered_a", "index_a", "gathered_b",
                                                              "index_b", "index_c"]


def test_dispatcher_entry_points_keep_the_reference_names():
    from fastmd_amd.engine.dispatch import OpDispatcher

    # dispatch.py:349-350, :371, :545, :308, :301, :524, :532, :318, :340
    expect = {
        "segment_sum_graph": ["self", "value", "segment", "num_segment", "graph", "side", "weight", "bin_count"],
        "segment_sum": ["self", "value", "segment", "num_segment", "weight", "bin_count"],
        "gather_cat": ["self", "aligned", "gathered", "indices"],
        "use_csr_segment_sum": ["self", "value", "segment", "weight"],
        "use_weighted_segment_sum": ["self", "weight", "value"],
        "use_gather_cat": ["self", "aligned", "gathered"],
        "use_gather_cat4": ["self", "aligned", "gathered_a", "gathered_b"],
        "prepare_segment_csr": ["self", "graph", "num_segment"],
        "segment_csr": ["self", "graph", "side", "segment", "num_segment"],
        "pair_expand": ["self", "data", "directed2undirected", "graph"],
        "pair_average": ["self", "data", "directed2undirected", "graph"],
        "gather": ["self", "value", "indices"],
    }
    for name, args in expect.items():
        params = _params(getattr(OpDispatcher, name))
        assert [p.name for p in params] == args, name
    kw = {p.name for p in _params(OpDispatcher.segment_sum_graph) if p.kind == p.KEYWORD_ONLY}
    assert kw == {"weight", "bin_count"}


def test_dispatcher_has_one_path_and_refuses_cpu_tensors():
    import torch

    from fastmd_amd.engine.dispatch import OpDispatcher, dispatcher_for

    d = OpDispatcher()
    assert d.segment_sum_csr_enabled
    value = torch.ones(4, 3)
    seg = torch.tensor([0, 0, 1, 1])
    assert not d.use_csr_segment_sum(value, seg, None)  # CPU tensors: the HIP kernels do not take them
    with pytest.raises(ValueError, match="GPU tensor"):
        d.segment_sum(value, seg, 2)
    with pytest.raises(ValueError, match="GPU tensor"):
        d.segment_sum_graph(value, seg, 2, {"source_index": seg, "target_index": seg}, "target")
    with pytest.raises(ValueError, match="GPU tensor"):
        d.gather_cat(value, (value,), (seg, seg))

    class _Layout:
        route = "all_to_all"

    with pytest.raises(ValueError, match="single-device"):
        OpDispatcher(None, _Layout())
    assert dispatcher_for() is dispatcher_for()


def test_builder_defaults_are_the_reference_ones():
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder
    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder
    import torch

    # fixed_capacity_builder.py:1047-1070: t_capacity has no default, line graph at 4.5 A, padding None (sink atoms)
    sig = inspect.signature(FixedCapacityGraphBuilder.__init__).parameters
    assert sig["t_capacity"].default is inspect.Parameter.empty
    assert sig["line_graph_cutoff"].default == 4.5
    assert sig["padding"].default is None and sig["n_dummy"].default == 64
    with pytest.raises(TypeError, match="t_capacity"):
        FixedCapacityGraphBuilder(cell=torch.eye(3) * 20, atomic_numbers=torch.ones(2), u_capacity=8)
    # gpu_graph_builder.py:953: the ragged builder's default is a 4.5 A line graph, which it does not build
    assert inspect.signature(TensorGraphBuilder.__init__).parameters["line_graph_cutoff"].default == 4.5
    with pytest.raises(NotImplementedError, match="line_graph_cutoff=None"):
        TensorGraphBuilder(cell=torch.eye(3) * 20, atomic_numbers=torch.ones(2))


def test_dispatch_alias_resolves():
    import importlib

    from fastmd_amd.aliases import install_fastmd_aliases, uninstall_fastmd_aliases

    install_fastmd_aliases()
    try:
        module = importlib.import_module("fastmd.engine.dispatch")
        assert module.OpDispatcher.__module__ == "fastmd_amd.engine.dispatch"
        assert hasattr(module, "attach_dispatcher") and hasattr(module, "dispatcher_for")
    finally:
        uninstall_fastmd_aliases()


def _edges(n_cells=3):
    s = systems.perovskite(n_cells)
    cell32 = s.cell.astype(np.float32)
    inv = np.linalg.inv(s.cell).astype(np.float32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, np.float32(36.0 + 1e-3), 64)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(np.float32), wraps, np.float32(36.0),
                  np.float32(1.0), (1, 0, 0), 10 ** 8)
    e = b.n_edges
    return s.n_atoms, b.center[:e].astype(np.int64), b.neighbor[:e].astype(np.int64), b.edge_offsets


@pytest.mark.gpu
@pytest.mark.parametrize("shared", [False, True])
def test_aligned_gather_cat4_as_the_dispatcher_calls_it(device, shared):
    """``aligned_gather_cat4(aligned, gathered_a, index_a, gathered_b, index_b, index_c)``
    exactly as dispatch.py:555 calls it: forward bitwise ``torch.cat`` of the index selects,
    VJP within 1e-5 of the float64 scatter sums."""
    import torch

    from fastmd_amd.ops.gather_cat import aligned_gather_cat4

    print(f"[gather_cat4] shared={shared}", flush=True)
    g = torch.Generator().manual_seed(4)
    rows, na, nb, width = 3001, 517, 129, 64
    aligned = torch.randn(rows, width, generator=g)
    ga = torch.randn(na, width, generator=g)
    gb = ga if shared else torch.randn(nb, width, generator=g)
    nb = gb.shape[0]
    ia = torch.randint(0, na, (rows,), generator=g)
    ib = torch.randint(0, nb, (rows,), generator=g)
    ic = torch.randint(0, nb, (rows,), generator=g)
    ad = aligned.to(device).requires_grad_()
    gad = ga.to(device).requires_grad_()
    gbd = gad if shared else gb.to(device).requires_grad_()
    out = aligned_gather_cat4(ad, gad, ia.to(device), gbd, ib.to(device), ic.to(device))
    ref = torch.cat([ad, torch.index_select(gad, 0, ia.to(device)), torch.index_select(gbd, 0, ib.to(device)),
                     torch.index_select(gbd, 0, ic.to(device))], 1)
    assert out.shape == (rows, 4 * width)
    assert torch.equal(out, ref)
    gout = torch.randn(rows, 4 * width, generator=g)
    grads = torch.autograd.grad(out, [ad, gad] if shared else [ad, gad, gbd], gout.to(device))
    go = gout.double().numpy()
    assert torch.equal(grads[0].cpu(), gout[:, :width])
    ga_ref = oops.segment_sum(go[:, width:2 * width], ia.numpy(), na)
    gb_ref = (oops.segment_sum(go[:, 2 * width:3 * width], ib.numpy(), nb)
              + oops.segment_sum(go[:, 3 * width:], ic.numpy(), nb))
    if shared:
        assert oops.relative(grads[1].cpu().numpy(), ga_ref + gb_ref) < 1e-5
    else:
        assert oops.relative(grads[1].cpu().numpy(), ga_ref) < 1e-5
        assert oops.relative(grads[2].cpu().numpy(), gb_ref) < 1e-5


@pytest.mark.gpu
def test_dispatcher_gather_cat_both_arities(device):
    import torch

    from fastmd_amd.engine.dispatch import OpDispatcher

    d = OpDispatcher()
    g = torch.Generator().manual_seed(5)
    a = torch.randn(700, 32, generator=g).to(device)
    x = torch.randn(90, 32, generator=g).to(device)
    y = torch.randn(40, 32, generator=g).to(device)
    i = [torch.randint(0, 90, (700,), generator=g).to(device), torch.randint(0, 40, (700,), generator=g).to(device),
         torch.randint(0, 40, (700,), generator=g).to(device)]
    assert d.use_gather_cat(a, x) and d.use_gather_cat4(a, x, y)
    out3 = d.gather_cat(a, [x], [i[0], i[0]])
    assert torch.equal(out3, torch.cat([a, x[i[0]], x[i[0]]], 1))
    out4 = d.gather_cat(a, (x, y), (i[0], i[1], i[2]))
    assert torch.equal(out4, torch.cat([a, x[i[0]], y[i[1]], y[i[2]]], 1))
    assert torch.equal(d.gather(x, i[0]), x[i[0]])
    with pytest.raises(ValueError, match="gathered"):
        d.gather_cat(a, (x, y), (i[0], i[1]))


@pytest.mark.gpu
def test_dispatcher_segment_sum_graph_both_sides(device):
    """``OpDispatcher().segment_sum_graph`` over the source (sender) and target (receiver)
    side of a perovskite edge graph against float64 sums, with and without a weight; the
    certified identity CSR of the sorted target side and the plain ``segment_sum`` give the
    same bits as the sorted CSR."""
    import torch

    from fastmd_amd.engine.dispatch import OpDispatcher

    print("[dispatch] segment_sum_graph 135 atoms", flush=True)
    n, center, neighbor, off = _edges(3)
    e = center.size
    g = torch.Generator().manual_seed(6)
    value = torch.randn(e, 48, generator=g)
    weight = torch.randn(e, 48, generator=g)
    d = OpDispatcher()
    graph = {"source_index": torch.tensor(neighbor, device=device), "target_index": torch.tensor(center, device=device),
             "_topology_graph_kind": "atom"}
    d.prepare_segment_csr(graph, n)
    for side, seg in (("source", neighbor), ("target", center)):
        vd = value.to(device).requires_grad_()
        wd = weight.to(device).requires_grad_()
        out = d.segment_sum_graph(vd, graph[f"{side}_index"], n, graph, side)
        assert oops.relative(out.detach().cpu().numpy(), oops.segment_sum(value.numpy(), seg, n)) < 1e-5
        outw = d.segment_sum_graph(vd, graph[f"{side}_index"], n, graph, side, weight=wd)
        assert oops.relative(outw.detach().cpu().numpy(),
                             oops.segment_sum(value.numpy(), seg, n, weight=weight.numpy())) < 1e-5
        gout = torch.randn(n, 48, generator=g)
        gv, gw = torch.autograd.grad(outw, [vd, wd], gout.to(device))
        gv_ref, gw_ref = oops.segment_sum_vjp(gout.numpy(), seg, weight=weight.numpy(), value=value.numpy())
        assert oops.relative(gv.cpu().numpy(), gv_ref) < 1e-5
        assert oops.relative(gw.cpu().numpy(), gw_ref) < 1e-5
        plain = d.segment_sum(vd.detach(), graph[f"{side}_index"], n)
        assert torch.equal(plain, out.detach())
        # a weight broadcast from [rows, 1] goes through segment_sum
        w1 = weight[:, :1].contiguous()
        out1 = d.segment_sum_graph(vd.detach(), graph[f"{side}_index"], n, graph, side, weight=w1.to(device))
        assert oops.relative(out1.cpu().numpy(),
                             oops.segment_sum(value.numpy(), seg, n, weight=np.repeat(w1.numpy(), 48, 1))) < 1e-5

    class _Sorted:
        route = "identity"
        identity_csr = ("atom",)

    sorted_graph = {"source_index": graph["source_index"], "target_index": graph["target_index"],
                    "_topology_graph_kind": "atom",
                    "_target_segment_attention_counts": torch.tensor(np.diff(off[:n + 1]), device=device)}
    ds = OpDispatcher(None, _Sorted())
    ds.prepare_segment_csr(sorted_graph, n)
    perm, offs, identity, skip = sorted_graph["_target_segment_sum_csr"]
    assert identity and perm is None and skip == -1
    assert torch.equal(offs.cpu(), torch.tensor(off[:n + 1], dtype=torch.int64))
    vd = value.to(device)
    assert torch.equal(ds.segment_sum_graph(vd, sorted_graph["target_index"], n, sorted_graph, "target"),
                       d.segment_sum_graph(vd, graph["target_index"], n, graph, "target"))


@pytest.mark.gpu
def test_dispatcher_pairs_and_attach(device):
    import torch

    from fastmd_amd.engine.dispatch import OpDispatcher, attach_dispatcher

    g = torch.Generator().manual_seed(7)
    u = 200
    d2u = torch.randperm(2 * u, generator=g) % u  # each pair twice
    data = torch.randn(u, 16, generator=g)
    d = OpDispatcher()
    graph = {"num_undirected": u}
    expanded = d.pair_expand(data.to(device), d2u.to(device), graph)
    assert torch.equal(expanded.cpu(), data[d2u])
    rows = torch.randn(2 * u, 16, generator=g)
    avg = d.pair_average(rows.to(device), d2u.to(device), graph)
    ref = oops.segment_sum(rows.numpy(), d2u.numpy(), u) / 2.0
    assert oops.relative(avg.cpu().numpy(), ref) < 1e-6
    atom = {"source_index": torch.tensor([1, 0, 2], device=device), "target_index": torch.tensor([0, 1, 1], device=device),
            "num_segment": 3, "num_undirected": 2}
    line = {}
    batch = {"atom_graph_dict": atom, "line_graph_dict": line}
    disp = attach_dispatcher(batch)
    assert batch["_ops"] is disp and atom["_ops"] is disp and line["_ops"] is disp
    assert "_source_segment_sum_csr" in atom and "_target_segment_sum_csr" in atom


@pytest.mark.gpu
def test_builder_reference_defaults_build_a_sink_padded_line_graph(device):
    """A reference caller passing only ``t_capacity`` gets the 4.5 A line graph with sink padding
    (64 sinks): bitwise the build with those arguments spelled out."""
    import torch

    from fastmd_amd.adapters.protocol import PaddingRule
    from fastmd_amd.graph.fixed_capacity_builder import FixedCapacityGraphBuilder

    s = systems.perovskite(3)
    # 4.5 A bonds: 12 per atom and about 19 000 triplets in the 135-atom cell
    common = dict(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers), u_capacity=1200,
                  t_capacity=24000, atom_graph_cutoff=6.0, candidate_cutoff=8.0, device=device)
    default = FixedCapacityGraphBuilder(**common)
    spelled = FixedCapacityGraphBuilder(line_graph_cutoff=4.5, padding=PaddingRule("sink_atoms"), n_dummy=64, **common)
    assert default.line_graph_cutoff == 4.5 and default.padding.kind == "sink_atoms" and default.n_dummy == 64
    pos = torch.tensor(s.positions, device=device)
    _, status = default.build(pos, rebuild_candidates=True)
    spelled.build(pos, rebuild_candidates=True)
    assert 0 < int(status.triplet_count.item()) <= 24000 and not bool(status.overflow.item())
    for name in ("edge_index", "edge_image", "n_edges", "pair_d2u", "pair_u2d", "triplets"):
        a, b = getattr(default.batch, name), getattr(spelled.batch, name)
        assert torch.equal(a, b), name
    assert int(default.batch.n_edges.item()) > 0


def _integration_stub():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = re.search(r"```python\n(# fastmd/engine/kernels/hip_backend\.py.*?)```", text, re.S)
    assert block is not None, "the integration guide lost its reference-side binding"
    return block.group(1)


def test_integration_stub_binds_the_header_signatures():
    """The argtypes the reference-side binding sets are the library's own (the ctypes table that
    mirrors include/fastmd_hip.h)."""
    from fastmd_amd import _abi

    src = _integration_stub()
    aliases = {"_p": "_p", "_i32": "_i32", "_i64": "_i64", "_f32": "_f32"}
    found = re.findall(r"_lib\.(fmd_\w+)\.argtypes = \[([^\]]*)\]", src)
    assert {name for name, _ in found} >= {"fmd_segsum_csr_f32", "fmd_gather_cat_f32", "fmd_gemm_f32"}
    for name, args in found:
        stub = [getattr(_abi, aliases[a.strip()]) for a in args.split(",")]
        assert stub == _abi.SIGNATURES[name][1], name


@pytest.mark.gpu
def test_integration_stub_runs(device):
    """The integration guide's binding, executed as written (library path filled in): its segment sum,
    4-part gather-cat and linear agree with this build's operators."""
    import torch

    from fastmd_amd import _abi
    from fastmd_amd.ops.csr_segment_sum import csr_segment_sum
    from fastmd_amd.ops.wide_gemm import linear

    src = _integration_stub().replace('"libfastmd_hip.so"', repr(_abi.LIB_PATH))
    ns: dict = {}
    exec(compile(src, "INTEGRATION.md:hip_backend", "exec"), ns)
    n, center, neighbor, off = _edges(3)
    g = torch.Generator().manual_seed(8)
    value = torch.randn(center.size, 32, generator=g).to(device)
    offd = torch.tensor(off[:n + 1], dtype=torch.int64, device=device)
    out = ns["csr_segment_sum_hip"](value, offd, n)
    ref = csr_segment_sum(value, torch.tensor(center, device=device), n, None, offd, True)
    assert torch.equal(out, ref)
    a = torch.randn(300, 16, generator=g).to(device)
    x = torch.randn(50, 16, generator=g).to(device)
    y = torch.randn(20, 16, generator=g).to(device)
    ia, ib, ic = (torch.randint(0, m, (300,), generator=g).to(device) for m in (50, 20, 20))
    assert torch.equal(ns["aligned_gather_cat4_hip"](a, x, ia, y, ib, ic), torch.cat([a, x[ia], y[ib], y[ic]], 1))
    xs = torch.randn(1000, 136, generator=g).to(device)
    w = torch.randn(512, 136, generator=g).to(device)
    bias = torch.randn(512, generator=g).to(device)
    ys = ns["linear_hip"](xs, w, bias)
    assert oops.relative(ys.cpu().numpy(), oops.linear(xs.cpu().numpy(), w.cpu().numpy(), bias.cpu().numpy())) < 1e-5
    assert torch.equal(ys, linear(xs, w, bias))
