"""(b) gather-cat, (c) CSR segment sums, (d) MFMA GEMM: HIP kernels vs the oracle."""
import functools

import numpy as np
import pytest

from oracle import ops as oops
from oracle import nl as onl
from fastmd_amd import systems


def test_relative_metric():
    assert oops.relative([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert oops.relative([1.0, 2.5], [1.0, 2.0]) == pytest.approx(0.25)


def test_oracle_segment_sum_closed_form():
    value = np.arange(12, dtype=np.float64).reshape(6, 2)
    seg = np.array([0, 0, 2, 2, 2, 1])
    out = oops.segment_sum(value, seg, 3)
    assert np.array_equal(out, [[2, 4], [10, 11], [18, 21]])
    gv, gw = oops.segment_sum_vjp(np.ones((3, 2)) * [[1], [2], [3]], seg, weight=2.0, value=value)
    assert np.array_equal(gv[:, 0], [2, 2, 6, 6, 6, 4])


@functools.lru_cache(maxsize=2)
def _edge_list(n_atoms=135, cutoff=6.0):
    s = systems.perovskite_atoms(n_atoms)
    cell32 = s.cell.astype(np.float32)
    inv = np.linalg.inv(s.cell).astype(np.float32)
    _, wraps, wrapped = onl.wrap(s.positions, inv, cell32)
    cand = onl.candidates(wrapped, cell32, np.float32(cutoff ** 2 + 1e-3), 64)
    b = onl.build(s.positions, inv, cell32, cand, s.positions.astype(np.float32), wraps, np.float32(cutoff ** 2),
                  np.float32(1.0), (1, 0, 0), 10 ** 8)
    e = b.n_edges
    rev = onl.reverse(b.center, b.neighbor, b.images, b.edge_offsets, e)
    return b.center[:e], b.neighbor[:e], b.edge_offsets, rev, wrapped, b.distances[:e]


@pytest.mark.gpu
@pytest.mark.parametrize("F", [64, 128, 256])
def test_gather_cat_forward_bitwise_and_vjp(device, F):
    import torch

    from fastmd_amd.ops.csr_segment_sum import Csr
    from fastmd_amd.ops.gather_cat import aligned_gather_cat3, gather_cat

    print(f"[gather_cat] F={F}", flush=True)
    center, neighbor, off, rev, _, dist = _edge_list()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(135, F, generator=g)
    rbf = torch.randn(center.size, 8, generator=g)
    src = torch.tensor(neighbor, dtype=torch.int32)
    dst = torch.tensor(center, dtype=torch.int32)
    xd, rbfd = x.to(device).requires_grad_(), rbf.to(device).requires_grad_()
    csr_dst = Csr(torch.tensor(off, device=device))
    csr_src = Csr(torch.tensor(off, device=device), torch.tensor(rev, device=device))
    out = gather_cat(xd, src.to(device), dst.to(device), rbfd, src_csr=csr_src, dst_csr=csr_dst)
    ref = oops.gather_cat([(x.numpy(), neighbor), (x.numpy(), center), (rbf.numpy(), None)])
    assert out.shape == (center.size, 2 * F + 8)
    assert np.array_equal(out.detach().cpu().numpy(), ref.astype(np.float32))
    gout = torch.randn(out.shape, generator=g)
    out.backward(gout.to(device))
    gx_ref = (oops.segment_sum(gout[:, :F].numpy(), neighbor, 135) + oops.segment_sum(gout[:, F:2 * F].numpy(), center, 135))
    assert oops.relative(xd.grad.cpu().numpy(), gx_ref) < 1e-6
    assert np.array_equal(rbfd.grad.cpu().numpy(), gout[:, 2 * F:].numpy())
    # deterministic: the same VJP twice, bitwise
    g1 = xd.grad.clone()
    xd.grad = None
    gather_cat(xd, src.to(device), dst.to(device), rbfd, src_csr=csr_src, dst_csr=csr_dst).backward(gout.to(device))
    assert torch.equal(g1, xd.grad)
    # reference form, CSRs built from the indices
    aligned = torch.randn(center.size, F, generator=g)
    a = aligned_gather_cat3(aligned.to(device), x.to(device), dst.to(device), src.to(device))
    assert np.array_equal(a.cpu().numpy(), oops.gather_cat([(aligned.numpy(), None), (x.numpy(), center),
                                                            (x.numpy(), neighbor)]).astype(np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("F", [1, 3, 64, 128, 256, 512])
def test_segment_sum_identity_and_perm_csr(device, F):
    import torch

    from fastmd_amd.ops.csr_segment_sum import Csr, csr_segment_sum, segment_sum_csr

    print(f"[segsum] F={F}", flush=True)
    center, neighbor, off, rev, _, _ = _edge_list()
    e = center.size
    g = torch.Generator().manual_seed(1)
    v = torch.randn(e, F, generator=g)
    w = torch.randn(e, F, generator=g)
    seg = torch.tensor(center, dtype=torch.int64)
    ref = oops.segment_sum(v.numpy(), center, 135)
    vd = v.to(device).requires_grad_()
    wd = w.to(device).requires_grad_()
    offd = torch.tensor(off, device=device)
    out = csr_segment_sum(vd, seg.to(device), 135, off=offd, identity_perm=True)
    assert oops.relative(out.detach().cpu().numpy(), ref) < 1e-5
    out2 = csr_segment_sum(vd, seg.to(device), 135, off=offd, identity_perm=True)
    assert torch.equal(out, out2)  # bitwise run to run
    # weighted, CSR built from the segment (permutation path), with the VJP
    outw = csr_segment_sum(vd, torch.tensor(neighbor, device=device), 135, weight=wd)
    refw = oops.segment_sum(v.numpy(), neighbor, 135, weight=w.numpy())
    assert oops.relative(outw.detach().cpu().numpy(), refw) < 1e-5
    gout = torch.randn(135, F, generator=g)
    outw.backward(gout.to(device))
    gv_ref, gw_ref = oops.segment_sum_vjp(gout.numpy(), neighbor, weight=w.numpy(), value=v.numpy())
    assert oops.relative(vd.grad.cpu().numpy(), gv_ref) < 1e-6
    assert oops.relative(wd.grad.cpu().numpy(), gw_ref) < 1e-6
    # two-term sum over the reverse CSR with a sign: sum_{src = i} v - sum_{dst = i} v
    both = segment_sum_csr([(v.to(device), Csr(offd, torch.tensor(rev, device=device)), 0, 1.0, None),
                            (v.to(device), Csr(offd), 0, -1.0, None)], 135, F)
    ref2 = oops.segment_sum(v.numpy(), neighbor, 135) - oops.segment_sum(v.numpy(), center, 135)
    assert oops.relative(both.cpu().numpy(), ref2) < 1e-5
    # skip_segment: zero output row and zero gradient for its rows
    vd.grad = None
    out3 = csr_segment_sum(vd, seg.to(device), 135, off=offd, identity_perm=True, skip_segment=7)
    assert float(out3[7].abs().max()) == 0.0
    out3.sum().backward()
    rows7 = center == 7
    assert float(vd.grad[torch.tensor(rows7, device=device)].abs().max()) == 0.0


def _segment_sums_f64(value, segment, n_segments):
    """fp64 sums of ``value`` rows by ``segment`` (stable sort, then one reduceat per run); every
    segment of the perovskite edge lists is non-empty."""
    order = np.argsort(segment, kind="stable")
    counts = np.bincount(segment, minlength=n_segments)
    assert counts.min() > 0
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    return np.add.reduceat(value[order].astype(np.float64), starts, axis=0)


@pytest.mark.gpu
@pytest.mark.parametrize("n_atoms", [3430, 40000])
@pytest.mark.parametrize("F", [64, 128, 256])
def test_ops_at_configs_sizes(device, n_atoms, F):
    """configs[1]'s sizes (N = 3 430 and 40 000, ~15 edges per atom at 6 A, F = 64 / 128 / 256),
    where the large-grid paths run: gather-cat bitwise equal to the concatenated row gathers and
    its VJP vs fp64 sums; the segment sum over the receiver CSR (identity permutation) and over the
    sender CSR (reverse-edge permutation) vs fp64 sums formed by sorting; the transpose bitwise
    equal to the row gather it is."""
    import torch

    from fastmd_amd.ops.csr_segment_sum import Csr, csr_segment_sum, segment_sum_t
    from fastmd_amd.ops.gather_cat import gather_cat

    print(f"[ops large] N={n_atoms} F={F}", flush=True)
    center, neighbor, off, rev, _, _ = _edge_list(n_atoms)
    e = center.size
    g = torch.Generator().manual_seed(F)
    x = torch.randn(n_atoms, F, generator=g)
    rbf = torch.randn(e, 8, generator=g)
    offd = torch.tensor(off, device=device)
    dst_csr, src_csr = Csr(offd), Csr(offd, torch.tensor(rev, device=device))
    src, dst = torch.tensor(neighbor, device=device), torch.tensor(center, device=device)
    xd = x.to(device).requires_grad_()
    out = gather_cat(xd, src, dst, rbf.to(device), src_csr=src_csr, dst_csr=dst_csr)
    xn = x.numpy()
    assert np.array_equal(out.detach().cpu().numpy(), np.concatenate([xn[neighbor], xn[center], rbf.numpy()], 1))
    gout = torch.randn(e, 2 * F + 8, generator=g)
    out.backward(gout.to(device))
    del out
    gx_ref = (_segment_sums_f64(gout[:, :F].numpy(), neighbor, n_atoms)
              + _segment_sums_f64(gout[:, F:2 * F].numpy(), center, n_atoms))
    assert oops.relative(xd.grad.cpu().numpy(), gx_ref) < 1e-6
    v = gout[:, :F].contiguous()
    vd = v.to(device)
    by_dst = csr_segment_sum(vd, dst, n_atoms, off=offd, identity_perm=True)
    assert oops.relative(by_dst.cpu().numpy(), _segment_sums_f64(v.numpy(), center, n_atoms)) < 1e-5
    by_src = csr_segment_sum(vd, src, n_atoms, off=offd, perm=src_csr.perm)
    assert oops.relative(by_src.cpu().numpy(), _segment_sums_f64(v.numpy(), neighbor, n_atoms)) < 1e-5
    node = torch.randn(n_atoms, F, generator=g)
    gv, _ = segment_sum_t(node.to(device), dst_csr, e)
    assert np.array_equal(gv.cpu().numpy(), node.numpy()[center])
    gv_src, _ = segment_sum_t(node.to(device), src_csr, e)
    assert np.array_equal(gv_src.cpu().numpy(), node.numpy()[neighbor])


@pytest.mark.gpu
def test_segment_sum_padding_rows_excluded(device):
    """Rows past off[-1] (fixed-capacity padding) add nothing and get zero gradient."""
    import torch

    from fastmd_amd.ops.csr_segment_sum import csr_segment_sum

    off = torch.tensor([0, 2, 3], device=device)
    v = torch.arange(10.0, device=device).reshape(5, 2).requires_grad_()
    out = csr_segment_sum(v, None, 2, off=off, identity_perm=True)
    assert out.tolist() == [[2.0, 4.0], [4.0, 5.0]]
    out.sum().backward()
    assert v.grad.tolist() == [[1, 1], [1, 1], [1, 1], [0, 0], [0, 0]]


@pytest.mark.gpu
@pytest.mark.parametrize("F", [64, 128, 256])
@pytest.mark.parametrize("m", [1, 100, 2054])
def test_gemm_fp32_against_fp64(device, F, m):
    import torch

    from fastmd_amd.ops.wide_gemm import edge_gemm, linear, matmul

    print(f"[gemm] F={F} m={m}", flush=True)
    g = torch.Generator().manual_seed(2)
    k, n = 2 * F + 8, 4 * F
    a = torch.randn(m, k, generator=g)
    w = torch.randn(k, n, generator=g) / k ** 0.5
    ref = a.double() @ w.double()
    y = edge_gemm(a.to(device), w.to(device))
    assert oops.relative(y.cpu().numpy(), ref.numpy()) < 1e-5
    wl = w.t().contiguous()  # F.linear layout [N, K]
    b = torch.randn(n, generator=g)
    ad = a.to(device).requires_grad_()
    yl = linear(ad, wl.to(device), b.to(device))
    assert oops.relative(yl.detach().cpu().numpy(), (ref + b.double()).numpy()) < 1e-5
    gy = torch.randn(m, n, generator=g)
    yl.backward(gy.to(device))
    assert oops.relative(ad.grad.cpu().numpy(), (gy.double() @ wl.double()).numpy()) < 1e-5
    mm = matmul(gy.to(device), wl.to(device))
    assert oops.relative(mm.cpu().numpy(), (gy.double() @ wl.double()).numpy()) < 1e-5
    ys = edge_gemm(a.to(device), w.to(device), epilogue="silu")
    assert oops.relative(ys.cpu().numpy(), torch.nn.functional.silu(ref).numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("b_layout", [0, 1])
def test_gemm_thin_shapes_against_fp64(device, b_layout):
    """fmd_gemm_f32 on K <= 16 (outer-product form) and N <= 16 (row-dot form): ragged M, every K
    bucket, N up to 256, a row pitch that is not a multiple of 4 (scalar loads), bias, accumulate
    and the SiLU epilogue, within 1e-6 of float64 (fp32 FMA chains; 1e-5 past K = 256, where K = 1 000
    with N = 16 exceeds the row-dot form's LDS and takes the matrix-core path); rows are independent
    of the launch's other rows (the same bits for a slice) and run-to-run bitwise."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    g = torch.Generator().manual_seed(21)
    shapes = [(1, 1, 1), (37, 3, 5), (1000, 8, 64), (38401, 9, 256), (777, 16, 200), (500, 12, 130),
              (100, 3, 9), (5000, 64, 8), (38401, 256, 9), (333, 800, 16), (333, 1000, 16), (777, 130, 4),
              (64, 17, 1)]
    for i, (m, k, n) in enumerate(shapes):
        print(f"[gemm thin] m={m} k={k} n={n} layout={b_layout}", flush=True)
        a = torch.randn(m, k + 3, generator=g)[:, :k] if i % 3 == 2 else torch.randn(m, k, generator=g)
        w = torch.randn(k, n, generator=g) / k ** 0.5
        wb = w if b_layout == 1 else w.t().contiguous()
        bias = torch.randn(n, generator=g) if i % 2 else None
        c0 = torch.randn(m, n, generator=g)
        ref = a.double() @ w.double() + (bias.double() if bias is not None else 0.0)
        ad, wd = a.to(device), wb.to(device)
        bd = bias.to(device) if bias is not None else None
        tol = 1e-6 if k <= 256 else 1e-5
        y = gemm(ad, wd, b_layout=b_layout, bias=bd)
        assert oops.relative(y.cpu().numpy(), ref.numpy()) < tol
        assert torch.equal(gemm(ad, wd, b_layout=b_layout, bias=bd), y)
        ys = gemm(ad, wd, b_layout=b_layout, bias=bd, epilogue="silu")
        assert oops.relative(ys.cpu().numpy(), torch.nn.functional.silu(ref).numpy()) < tol
        out = c0.to(device)
        gemm(ad, wd, b_layout=b_layout, bias=bd, out=out, accumulate=True)
        assert oops.relative(out.cpu().numpy(), (ref + c0.double()).numpy()) < tol
        if m > 40:
            part = gemm(ad[13:40], wd, b_layout=b_layout, bias=bd)
            assert torch.equal(part, y[13:40])


@pytest.mark.gpu
def test_gemm_fp32_large_tiles(device):
    """The 10k-atom edge GEMM shape (ragged M, K = 2F+8, N = 4F) takes the 128x128 tile path:
    both B layouts, the bias/SiLU epilogue and accumulate against float64."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    g = torch.Generator().manual_seed(5)
    m, k, n = 66001, 264, 512
    a = torch.randn(m, k, generator=g)
    w = torch.randn(k, n, generator=g) / k ** 0.5
    bias = torch.randn(n, generator=g)
    ref = a.double() @ w.double()
    ad, wd = a.to(device), w.to(device)
    y = gemm(ad, wd, b_layout=1)
    assert oops.relative(y.cpu().numpy(), ref.numpy()) < 1e-5
    wt = w.t().contiguous().to(device)
    ys = gemm(ad, wt, b_layout=0, bias=bias.to(device), epilogue="silu")
    assert oops.relative(ys.cpu().numpy(), torch.nn.functional.silu(ref + bias.double()).numpy()) < 1e-5
    c0 = torch.randn(m, n, generator=g)
    out = c0.to(device)
    gemm(ad, wd, b_layout=1, out=out, accumulate=True)
    assert oops.relative(out.cpu().numpy(), (ref + c0.double()).numpy()) < 1e-5
    # the VJP shape (N = 2F+8: a partial last N tile) and a row pitch that is not a multiple of 4
    # (masked loads on every K slice)
    gz = torch.randn(m, n, generator=g)
    gref = gz.double() @ w.double().t()
    gy = gemm(gz.to(device), wd, b_layout=0)
    assert oops.relative(gy.cpu().numpy(), gref.numpy()) < 1e-5
    wide = torch.zeros(m, k + 3)
    wide[:, :k] = a
    aw = wide.to(device)[:, :k]
    yw = gemm(aw, wt, b_layout=0)
    assert oops.relative(yw.cpu().numpy(), ref.numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("b_layout", [0, 1])
def test_gemm_group_matches_single_gemms_and_fp64(device, b_layout, monkeypatch):
    """fmd_gemm_group_f32: four problems of mixed shapes (ragged M, an empty one, a K split
    [a | a2], accumulate and bias) in one launch, each bitwise equal to the same problem through
    fmd_gemm_f32's 64 x 64 kernel (same K order) and within fp32 of float64 (groups this small
    otherwise take the K-split form: switched off here)."""
    import torch

    from fastmd_amd.ops import wide_gemm
    from fastmd_amd.ops.wide_gemm import gemm, gemm_group

    monkeypatch.setattr(wide_gemm, "GROUP_KS_MAX_TILES", 0)

    g = torch.Generator().manual_seed(11)

    def weight(k, n):
        w = torch.randn(k, n, generator=g) / k ** 0.5
        return w if b_layout == 1 else w.t().contiguous()  # stored [K, N] or [N, K]

    def ref_of(a, w):
        wk = w if b_layout == 1 else w.t()
        return a.double() @ wk.double()

    shapes = [(135, 128, 128), (405, 128, 128), (0, 128, 64), (1000, 64, 192)]
    probs, refs, singles = [], [], []
    for (m, k, n) in shapes:
        a = torch.randn(m, k, generator=g)
        w = weight(k, n)
        ref = ref_of(a, w)
        out = torch.empty(m, n, device=device)
        probs.append({"a": a.to(device), "b": w.to(device), "out": out})
        refs.append(ref)
        singles.append(gemm(a.to(device), w.to(device), b_layout=b_layout))
    # accumulate + bias on the last problem
    c0 = torch.randn(1000, 192, generator=g)
    bias = torch.randn(192, generator=g)
    probs[3]["out"] = c0.to(device)
    probs[3]["accumulate"] = True
    probs[3]["bias"] = bias.to(device)
    refs[3] = refs[3] + c0.double() + bias.double()
    out_single = c0.to(device)
    gemm(probs[3]["a"], probs[3]["b"], b_layout=b_layout, out=out_single, accumulate=True, bias=bias.to(device))
    singles[3] = out_single
    gemm_group(probs, b_layout=b_layout)
    for p, ref, single in zip(probs, refs, singles):
        assert torch.equal(p["out"], single)
        if ref.numel():
            assert oops.relative(p["out"].cpu().numpy(), ref.numpy()) < 1e-5
    # K split: [a | a2] @ [W0; W1] in one accumulation
    m, k1, k2, n = 777, 128, 128, 128
    a, a2 = torch.randn(m, k1, generator=g), torch.randn(m, k2, generator=g)
    w = weight(k1 + k2, n)
    out = torch.empty(m, n, device=device)
    gemm_group([{"a": a.to(device), "a2": a2.to(device), "b": w.to(device), "out": out}], b_layout=b_layout)
    single = gemm(torch.cat([a, a2], 1).to(device), w.to(device), b_layout=b_layout)
    assert torch.equal(out, single)
    assert oops.relative(out.cpu().numpy(), ref_of(torch.cat([a, a2], 1), w).numpy()) < 1e-5


@pytest.mark.gpu
def test_gemm_group_ks_form(device):
    """fmd_gemm_group_ks_f32 (small groups, B [N, K]: 16 x 16 tiles, K shared by four waves):
    ragged M and N, K = 4, 16, 136 (a partial last slice), 1 024 and a split [a | a2], accumulate,
    bias and the SiLU epilogue, each within fp32 of float64; every problem's result the same bits
    alone as in the group and on a second call; gemm_group picks it below GROUP_KS_MAX_TILES
    64 x 64 tiles and gemm_splitk for small products."""
    import torch

    from fastmd_amd.ops import wide_gemm
    from fastmd_amd.ops.wide_gemm import gemm_group, gemm_splitk

    g = torch.Generator().manual_seed(31)
    d = lambda t: t.to(device)  # noqa: E731
    shapes = [(135, 128, 512), (405, 136, 128), (1, 4, 16), (17, 16, 130)]
    mats = []
    for (m, k, n) in shapes:
        mats.append((torch.randn(m, k, generator=g), torch.randn(n, k, generator=g) / k ** 0.5))
    c3 = torch.randn(17, 130, generator=g)
    bias = torch.randn(128, generator=g)

    def problems():
        ps = [{"a": d(a), "b": d(w), "out": torch.empty(a.shape[0], w.shape[0], device=device)} for a, w in mats]
        ps[1]["bias"] = d(bias)
        ps[3]["out"] = d(c3)
        ps[3]["accumulate"] = True
        return ps

    ref = [a.double() @ w.double().t() for a, w in mats]
    ref[1] = ref[1] + bias.double()
    ref[3] = ref[3] + c3.double()
    runs = []
    for _ in range(2):
        ps = problems()
        gemm_group(ps, b_layout=0)
        runs.append([p["out"].clone() for p in ps])
    for out, r in zip(runs[0], ref):
        assert oops.relative(out.cpu().numpy(), r.numpy()) < 1e-5
    for x, y in zip(runs[0], runs[1]):
        assert torch.equal(x, y)
    for i, p in enumerate(problems()):
        gemm_group([p], b_layout=0)
        assert torch.equal(p["out"], runs[0][i])
    # the K-split form, not the 64 x 64 tiles: the same problems with the K-split form switched off
    # give other bits (a different K order)
    saved = wide_gemm.GROUP_KS_MAX_TILES
    try:
        wide_gemm.GROUP_KS_MAX_TILES = 0
        ps = problems()
        gemm_group(ps, b_layout=0)
        assert not torch.equal(ps[0]["out"], runs[0][0])
    finally:
        wide_gemm.GROUP_KS_MAX_TILES = saved
    # SiLU epilogue
    a, w = mats[0]
    out = torch.empty(135, 512, device=device)
    gemm_group([{"a": d(a), "b": d(w), "out": out}], b_layout=0, epilogue="silu")
    assert oops.relative(out.cpu().numpy(), torch.nn.functional.silu(ref[0]).numpy()) < 1e-5
    # [a | a2] with K = 512 + 512 through gemm_splitk (small: the K-split group), accumulate
    a1, a2 = torch.randn(135, 512, generator=g), torch.randn(135, 512, generator=g)
    w = torch.randn(128, 1024, generator=g) / 32.0
    c0 = torch.randn(135, 128, generator=g)
    outs = []
    for _ in range(2):
        out = d(c0)
        gemm_splitk(d(a1), d(w), b_layout=0, out=out, a2=d(a2), accumulate=True)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    r = torch.cat([a1, a2], 1).double() @ w.double().t() + c0.double()
    assert oops.relative(outs[0].cpu().numpy(), r.numpy()) < 1e-5
    # the split operand gives the concatenated operand's bits (the same slices in the same order),
    # and accumulating adds C to the same sum
    out = torch.empty(135, 128, device=device)
    gemm_group([{"a": d(a1), "a2": d(a2), "b": d(w), "out": out}], b_layout=0)
    out_cat = torch.empty(135, 128, device=device)
    gemm_group([{"a": d(torch.cat([a1, a2], 1)), "b": d(w), "out": out_cat}], b_layout=0)
    assert torch.equal(out, out_cat)
    assert torch.equal(out + d(c0), outs[0])


@pytest.mark.gpu
def test_gemm_group_split_plane_form(device):
    """A large fmd_gemm_group_f32 group with B [N, K] and the weights' planes (the node side of a
    layer at 10 000 atoms: >= 128 tiles of 128 x 128) runs as split-plane GEMMs
    (fmd_gemm_group_x3_planes_f32): each problem within fp32 of float64 and bitwise equal to
    fmd_gemm_f32's split-plane kernel on the same problem (M large enough that it takes that
    kernel; a K split at 128 gives the concatenated operand's bits), in the 64-row and the 128-row
    tile forms. Without planes the group keeps the fp32 tiles."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm, gemm_group, split_planes

    g = torch.Generator().manual_seed(12)
    C = 128
    a0, a1 = torch.randn(33000, C, generator=g), torch.randn(33000, C, generator=g)
    w0 = torch.randn(C, C, generator=g) / C ** 0.5
    w1 = torch.randn(C, 2 * C, generator=g) / (2 * C) ** 0.5  # [N, K]: [a0 | a1] W1^T
    c1 = torch.randn(33000, C, generator=g)
    bias = torch.randn(C, generator=g)
    d = lambda t: t.to(device)  # noqa: E731
    out0 = torch.empty(33000, C, device=device)
    out1 = d(c1)
    gemm_group([{"a": d(a0), "b": d(w0), "b_planes": split_planes(d(w0)), "out": out0},
                {"a": d(a0), "a2": d(a1), "b": d(w1), "b_planes": split_planes(d(w1)), "out": out1,
                 "accumulate": True, "bias": d(bias)}], b_layout=0)
    ref0 = a0.double() @ w0.double().t()
    ref1 = torch.cat([a0, a1], 1).double() @ w1.double().t() + c1.double() + bias.double()
    assert oops.relative(out0.cpu().numpy(), ref0.numpy()) < 1e-5
    assert oops.relative(out1.cpu().numpy(), ref1.numpy()) < 1e-5
    assert torch.equal(out0, gemm(d(a0), d(w0), b_layout=0))
    single = d(c1)
    gemm(d(torch.cat([a0, a1], 1)), d(w1), b_layout=0, out=single, accumulate=True, bias=d(bias))
    assert torch.equal(out1, single)
    # 128-row tiles once a group has eight per CU (2 188 here): the same bits as the 64-row form
    a2 = torch.randn(140000, C, generator=g)
    w2 = torch.randn(2 * C, C, generator=g) / C ** 0.5
    out2 = torch.empty(140000, 2 * C, device=device)
    gemm_group([{"a": d(a2), "b": d(w2), "b_planes": split_planes(d(w2)), "out": out2}], b_layout=0)
    assert torch.equal(out2, gemm(d(a2), d(w2), b_layout=0))
    assert torch.equal(out2[:33000], gemm(d(a2[:33000]), d(w2), b_layout=0))
    assert oops.relative(out2.cpu().numpy(), (a2.double() @ w2.double().t()).numpy()) < 1e-5
    # without planes: the fp32 tiles (within fp32 rounding of the same product, not its bits)
    out0f = torch.empty(33000, C, device=device)
    gemm_group([{"a": d(a0), "b": d(w0), "out": out0f}], b_layout=0)
    assert oops.relative(out0f.cpu().numpy(), ref0.numpy()) < 1e-5
    assert not torch.equal(out0f, out0)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [33000, 3000, 200])
def test_gemm_group_row_add_is_a_prefill(device, m):
    """gemm_group's row_add (row index[r] of a table added to output row r): on the split-plane
    form (fmd_gemm_group_x3_planes_rows_f32, the rows added in the epilogue; m = 33 000), on the
    fp32 grouped tiles (no planes) and on the small K-split form (m = 200) bitwise the result of
    prefilling the output with those rows (fmd_embed_f32) and accumulating; a problem without
    row_add in the same group is unchanged; within fp32 of float64."""
    import torch

    from fastmd_amd import _abi
    from fastmd_amd.ops.wide_gemm import gemm_group, split_planes

    print(f"[row_add] m={m}", flush=True)
    g = torch.Generator().manual_seed(m)
    C = 128
    d = lambda t: t.to(device)  # noqa: E731
    a = d(torch.randn(m, C, generator=g))
    w0 = d(torch.randn(C, C, generator=g) / C ** 0.5)
    w1 = d(torch.randn(4 * C, C, generator=g) / C ** 0.5)
    tab0 = d(torch.randn(3, C, generator=g))
    tab1 = d(torch.randn(5, 4 * C, generator=g))
    idx = d(torch.randint(0, 3, (m,), generator=g, dtype=torch.int32))
    idx1 = d(torch.randint(0, 5, (m,), generator=g, dtype=torch.int32))
    for planes in (True, False):
        o0, o1, o2 = torch.empty(m, C, device=device), torch.empty(m, 4 * C, device=device), torch.empty(m, C,
                                                                                                       device=device)
        probs = [{"a": a, "b": w0, "out": o0, "row_add": (tab0, idx)}, {"a": a, "b": w1, "out": o1,
                                                                        "row_add": (tab1, idx1)},
                 {"a": a, "b": w0, "out": o2}]
        if planes:
            for p in probs:
                p["b_planes"] = split_planes(p["b"])
        gemm_group(probs, b_layout=0)
        p0, p1, p2 = torch.empty_like(o0), torch.empty_like(o1), torch.empty_like(o2)
        for tab, ix, out in ((tab0, idx, p0), (tab1, idx1, p1)):
            _abi.call("fmd_embed_f32", ix.data_ptr(), tab.data_ptr(), m, tab.shape[1], out.data_ptr(),
                      _abi.stream_handle(device))
        refs = [{"a": a, "b": w0, "out": p0, "accumulate": True}, {"a": a, "b": w1, "out": p1, "accumulate": True},
                {"a": a, "b": w0, "out": p2}]
        if planes:
            for p in refs:
                p["b_planes"] = split_planes(p["b"])
        gemm_group(refs, b_layout=0)
        assert torch.equal(o0, p0) and torch.equal(o1, p1) and torch.equal(o2, p2)
        ref1 = a.cpu().double() @ w1.cpu().double().t() + tab1.cpu().double()[idx1.cpu().long()]
        assert oops.relative(o1.cpu().numpy(), ref1.numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("F", [64, 128])
def test_gemm_bf16_against_fp64_of_rounded_inputs(device, F):
    import torch

    from fastmd_amd.ops.wide_gemm import edge_gemm

    g = torch.Generator().manual_seed(3)
    m, k, n = 777, 2 * F + 8, 4 * F
    a = torch.randn(m, k, generator=g)
    w = torch.randn(k, n, generator=g) / k ** 0.5
    y = edge_gemm(a.to(device), w.to(device), dtype=torch.bfloat16)
    ref = a.bfloat16().double() @ w.bfloat16().double()  # products of bf16 values are exact in fp32
    assert oops.relative(y.cpu().numpy(), ref.numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(777, 136, 256), (1000, 72, 200), (4099, 264, 512), (300, 520, 1024),
                                   (129, 8, 130), (5, 40, 7)])
def test_gemm_bf16_direct_to_lds(device, m, k, n):
    """The direct-to-LDS bf16 kernel (K-contiguous operands, aligned rows, K % 8 == 0): K tails of
    8 / 16 / 24 past a 32-k slice, fewer slices than stages, ragged M and N, against fp64 of the
    bf16 values; bitwise the register-staged kernel (taken when a row stride is not a multiple of
    8 elements), with bias, accumulation and the SiLU epilogue."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    g = torch.Generator().manual_seed(m + k + n)
    a = torch.randn(m, k, generator=g).bfloat16()
    b = torch.randn(n, k, generator=g).bfloat16() / k ** 0.5
    bias = torch.randn(n, generator=g)
    ref = a.double() @ b.double().t()
    y = gemm(a.to(device), b.to(device), b_layout=0)
    assert oops.relative(y.cpu().numpy(), ref.numpy()) < 1e-5
    # the same operands at row strides of k + 4: the register-staged kernel
    a_pad = torch.zeros(m, k + 4, dtype=torch.bfloat16)
    a_pad[:, :k] = a
    b_pad = torch.zeros(n, k + 4, dtype=torch.bfloat16)
    b_pad[:, :k] = b
    a_s, b_s = a_pad.to(device)[:, :k], b_pad.to(device)[:, :k]
    assert torch.equal(gemm(a_s, b_s, b_layout=0), y)
    c0 = torch.randn(m, n, generator=g).to(device)
    for kw in ({"bias": bias.to(device)}, {"epilogue": "silu"}, {"accumulate": True}):
        out_d, out_s = c0.clone(), c0.clone()
        gemm(a.to(device), b.to(device), b_layout=0, out=out_d, **kw)
        gemm(a_s, b_s, b_layout=0, out=out_s, **kw)
        assert torch.equal(out_d, out_s), kw


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,n", [(40000, 264, 512), (33001, 136, 256), (32768, 40, 130), (50000, 272, 200),
                                   (140000, 264, 512), (131073, 136, 300), (40000, 520, 1024), (33001, 280, 200),
                                   (50000, 544, 130)])
def test_gemm_bf16_resident_b(device, m, k, n):
    """The resident-B bf16 kernel (at least 32 768 rows, K <= 544, aligned K-contiguous operands):
    K tails of 8 past a 16-k step, a ragged last row block and column slab, one slab or several,
    one or two slabs per workgroup (from 131 072 rows), and past K = 272 the two k-rounds form;
    against fp64 of the bf16 values on a row sample, and bitwise the register-staged kernel with
    bias, accumulation and the SiLU epilogue."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    g = torch.Generator().manual_seed(m + k + n)
    a = torch.randn(m, k, generator=g).bfloat16()
    b = torch.randn(n, k, generator=g).bfloat16() / k ** 0.5
    bias = torch.randn(n, generator=g)
    y = gemm(a.to(device), b.to(device), b_layout=0)
    rows = torch.cat([torch.arange(0, 700), torch.arange(m - 300, m)])
    ref = a[rows].double() @ b.double().t()
    assert oops.relative(y.cpu()[rows].numpy(), ref.numpy()) < 1e-5
    # row strides of k + 4: the register-staged kernel, the same k-steps in the same order
    a_pad = torch.zeros(m, k + 4, dtype=torch.bfloat16)
    a_pad[:, :k] = a
    a_s = a_pad.to(device)[:, :k]
    assert torch.equal(gemm(a_s, b.to(device), b_layout=0), y)
    c0 = torch.randn(m, n, generator=g).to(device)
    for kw in ({"bias": bias.to(device)}, {"epilogue": "silu"}, {"accumulate": True}):
        out_d, out_s = c0.clone(), c0.clone()
        gemm(a.to(device), b.to(device), b_layout=0, out=out_d, **kw)
        gemm(a_s, b.to(device), b_layout=0, out=out_s, **kw)
        assert torch.equal(out_d, out_s), kw


@pytest.mark.gpu
@pytest.mark.parametrize("F", [64, 128])
def test_gemm_gather_against_fp64(device, F):
    """The fused gather-cat + edge GEMM (fmd_gemm_gather_f32) on a real neighbour list: parts
    [x[src] | x[dst] | rbf] read through strided int32 columns of edge_index, against fp64 of
    torch.cat; the bias/SiLU and accumulate epilogues; and a layout the fused kernel declines
    (a first part of width 12) through the gather-then-GEMM fallback."""
    import numpy as np
    import torch

    from fastmd_amd import systems
    from fastmd_amd.graph.gpu_graph_builder import TensorGraphBuilder
    from fastmd_amd.ops.wide_gemm import gemm_gather

    print(f"[gemm_gather] F={F}", flush=True)
    s = systems.perovskite(4)
    g = TensorGraphBuilder(cell=torch.tensor(s.cell), atomic_numbers=torch.tensor(s.numbers), atom_graph_cutoff=6.0,
                           line_graph_cutoff=None, device=device).build(torch.tensor(s.positions, device=device))
    e = int(g.n_edges.item())
    ei = g.edge_index[:e]
    gen = torch.Generator().manual_seed(11)
    n_atoms = s.n_atoms
    x = torch.randn(n_atoms, F, generator=gen)
    rbf = torch.randn(e, 8, generator=gen)
    k, n = 2 * F + 8, 4 * F
    w = torch.randn(n, k, generator=gen) / k ** 0.5  # [N, K]
    eic = ei.cpu().long()
    a = torch.cat([x[eic[:, 1]], x[eic[:, 0]], rbf], 1).double()
    ref = a @ w.double().t()
    xd, rd, wd = x.to(device), rbf.to(device), w.to(device)
    z = gemm_gather([(xd, ei[:, 1]), (xd, ei[:, 0]), (rd, None)], wd)
    assert oops.relative(z.cpu().numpy(), ref.numpy()) < 1e-5
    bias = torch.randn(n, generator=gen)
    zs = gemm_gather([(xd, ei[:, 1]), (xd, ei[:, 0]), (rd, None)], wd, bias=bias.to(device), epilogue="silu")
    assert oops.relative(zs.cpu().numpy(), torch.nn.functional.silu(ref + bias.double()).numpy()) < 1e-5
    c0 = torch.randn(e, n, generator=gen)
    out = c0.to(device)
    gemm_gather([(xd, ei[:, 1]), (xd, ei[:, 0]), (rd, None)], wd, out=out, accumulate=True)
    assert oops.relative(out.cpu().numpy(), (ref + c0.double()).numpy()) < 1e-5
    # fallback layout: widths [12, 8] (the first is not a multiple of 16)
    x12 = torch.randn(n_atoms, 12, generator=gen)
    w2 = torch.randn(n, 20, generator=gen)
    ref2 = torch.cat([x12[eic[:, 0]], rbf], 1).double() @ w2.double().t()
    z2 = gemm_gather([(x12.to(device), ei[:, 0]), (rd, None)], w2.to(device))
    assert np.abs(z2.cpu().double().numpy() - ref2.numpy()).max() / np.abs(ref2.numpy()).max() < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("b_layout", [0, 1])
def test_gemm_splitk_against_fp64_and_run_to_run(device, b_layout):
    """fmd_gemm_splitk_f32: [a | a2] op(b) (+ bias) (+ C) with K in slices summed in slice order:
    within fp32 of float64 (ragged M and N), and bitwise the same on a second call."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm_splitk

    g = torch.Generator().manual_seed(23)
    m, k1, k2, n = 10001, 512, 512, 130
    a, a2 = torch.randn(m, k1, generator=g), torch.randn(m, k2, generator=g)
    w = torch.randn(k1 + k2, n, generator=g) / (k1 + k2) ** 0.5
    wb = w if b_layout == 1 else w.t().contiguous()
    c0 = torch.randn(m, n, generator=g)
    bias = torch.randn(n, generator=g)
    ref = torch.cat([a, a2], 1).double() @ w.double() + c0.double() + bias.double()
    outs = []
    for _ in range(2):
        out = c0.to(device)
        gemm_splitk(a.to(device), wb.to(device), b_layout=b_layout, out=out, a2=a2.to(device), bias=bias.to(device),
                    accumulate=True)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert oops.relative(outs[0].cpu().numpy(), ref.numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("m,ka,kb,n", [(10000, 512, 512, 128), (40000, 256, 256, 64), (20011, 1024, 0, 200)])
def test_gemm_splitk_split_planes(device, m, ka, kb, n):
    """fmd_gemm_splitk_x3_planes_f32 through gemm_splitk(b_planes=...): [a | a2] @ B^T with K cut
    into four slices of one grouped split-plane launch, summed in order, accumulate and bias:
    within 1e-5 of float64 and run-to-run bitwise (each split writes its own workspace slice)."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm_splitk, split_planes

    print(f"[splitk planes] m={m} ka={ka} kb={kb} n={n}", flush=True)
    g = torch.Generator().manual_seed(m + n)
    k = ka + kb
    a = torch.randn(m, ka, generator=g)
    a2 = torch.randn(m, kb, generator=g) if kb else None
    w = torch.randn(n, k, generator=g) / k ** 0.5
    bias = torch.randn(n, generator=g)
    c0 = torch.randn(m, n, generator=g)
    full = a if a2 is None else torch.cat([a, a2], 1)
    ref = full.double() @ w.double().t() + bias.double() + c0.double()
    wd = w.to(device)
    planes = split_planes(wd)
    outs = []
    for _ in range(2):
        out = c0.to(device)
        gemm_splitk(a.to(device), wd, b_layout=0, out=out, a2=a2.to(device) if a2 is not None else None,
                    bias=bias.to(device), accumulate=True, b_planes=planes)
        outs.append(out)
    assert oops.relative(outs[0].cpu().numpy(), ref.numpy()) < 1e-5
    assert torch.equal(outs[0], outs[1])


@pytest.mark.gpu
def test_gemm_planes_bitwise_equal_to_in_kernel_split(device):
    """fmd_split3_f32 gives x = p0 + p1 + p2 exactly (zero padding past the width), and the GEMM on
    pre-split planes (A gathered from plane rows, or fp32 A with pre-split B) is bitwise the GEMM
    that splits inside (same planes, products and order), including bias, accumulate and a
    gathered row add; and within fp32 of float64."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm_gather, gemm_planes, split_planes

    g = torch.Generator().manual_seed(21)
    n_atoms, E, C, nb, N = 3001, 40000, 128, 8, 512
    h0 = torch.randn(n_atoms, C, generator=g)
    ef = torch.randn(E, nb, generator=g) * 1e-3
    src = torch.randint(0, n_atoms, (E,), generator=g, dtype=torch.int32)
    w = torch.randn(N, C + nb, generator=g) / (C + nb) ** 0.5
    hp = split_planes(h0.to(device))
    total = hp.dense().double().sum(1)[:, :C].cpu()
    assert torch.equal(total, h0.double())
    efp = split_planes(ef.to(device))
    assert efp.ld == 48 and torch.equal(efp.dense().double().sum(1)[:, :nb].cpu(), ef.double())
    assert float(efp.dense()[:, :, nb:].abs().max()) == 0.0
    wp = split_planes(w.to(device))
    assert wp.ld == 48 * 9 and float(wp.dense()[:, :, C + nb:].abs().max()) == 0.0
    ref = gemm_gather([(h0.to(device), src.to(device)), (ef.to(device), None)], w.to(device))
    got = gemm_planes([(hp, src.to(device)), (efp, None)], wp, a_planes=True)
    assert torch.equal(got, ref)
    exact = torch.cat([h0[src.long()], ef], 1).double() @ w.double().t()
    assert oops.relative(got.cpu().numpy(), exact.numpy()) < 1e-5
    # bias + accumulate + gathered row add
    q = torch.randn(n_atoms, N, generator=g).to(device)
    qi = torch.randint(0, n_atoms, (E,), generator=g, dtype=torch.int32).to(device)
    c0 = torch.randn(E, N, generator=g).to(device)
    bias = torch.randn(N, generator=g).to(device)
    ref2 = gemm_gather([(h0.to(device), src.to(device)), (ef.to(device), None)], w.to(device), out=c0.clone(),
                       bias=bias, accumulate=True, row_add=(q, qi))
    got2 = gemm_planes([(hp, src.to(device)), (efp, None)], wp, a_planes=True, out=c0.clone(), bias=bias,
                       accumulate=True, row_add=(q, qi))
    assert torch.equal(got2, ref2)
    # fp32 A (split in the kernel) with pre-split B: the VJP shape [E, 4C] x [4C, C]
    gz = torch.randn(E, 4 * C, generator=g).to(device)
    wv = (torch.randn(C, 4 * C, generator=g) / (4 * C) ** 0.5).to(device)
    got3 = gemm_planes([(gz, None)], split_planes(wv), a_planes=False)
    assert torch.equal(got3, gemm_gather([(gz, None)], wv))


@pytest.mark.gpu
@pytest.mark.parametrize("C,nb,N,E", [(48, 8, 200, 3001), (64, 8, 256, 5000), (256, 8, 384, 4099)])
def test_gemm_planes_gathered_k_tails(device, C, nb, N, E):
    """The gathered pre-split GEMM over K = C + nb of 56, 72 and 264 (4, 5 and 17 slices of 16: the
    three-stage pipeline's loop and both tail lengths), ragged M and N: bitwise the in-kernel split
    and within fp32 of float64."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm_gather, gemm_planes, split_planes

    g = torch.Generator().manual_seed(C + N)
    n_atoms = 777
    h0 = torch.randn(n_atoms, C, generator=g)
    ef = torch.randn(E, nb, generator=g)
    src = torch.randint(0, n_atoms, (E,), generator=g, dtype=torch.int32)
    w = torch.randn(N, C + nb, generator=g) / (C + nb) ** 0.5
    d = lambda t: t.to(device)  # noqa: E731
    got = gemm_planes([(split_planes(d(h0)), d(src)), (split_planes(d(ef)), None)], split_planes(d(w)),
                      a_planes=True)
    ref = gemm_gather([(d(h0), d(src)), (d(ef), None)], d(w))
    assert torch.equal(got, ref)
    exact = torch.cat([h0[src.long()], ef], 1).double() @ w.double().t()
    assert oops.relative(got.cpu().numpy(), exact.numpy()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("N", [64, 40])
def test_gemm_gather_narrow_tile(device, N):
    """N <= 64 takes 128 x 64 split-plane tiles (the three-body model's edge rows): bitwise the
    columns of the same product on 128-wide tiles (the weight padded with more rows), and within
    fp32 of float64; with a gathered row add and accumulate."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm_gather

    g = torch.Generator().manual_seed(N)
    n_atoms, E, C = 500, 7001, 64
    h = torch.randn(n_atoms, C, generator=g)
    eps = torch.randn(E, C, generator=g)
    src = torch.randint(0, n_atoms, (E,), generator=g, dtype=torch.int32)
    w = torch.randn(N, 2 * C, generator=g) / (2 * C) ** 0.5
    wide = torch.cat([w, torch.randn(128 - N, 2 * C, generator=g)], 0)
    d = lambda t: t.to(device)  # noqa: E731
    got = gemm_gather([(d(h), d(src)), (d(eps), None)], d(w))
    ref = gemm_gather([(d(h), d(src)), (d(eps), None)], d(wide))[:, :N]
    assert torch.equal(got, ref)
    exact = torch.cat([h[src.long()], eps], 1).double() @ w.double().t()
    assert oops.relative(got.cpu().numpy(), exact.numpy()) < 1e-5
    q = torch.randn(n_atoms, N, generator=g)
    qi = torch.randint(0, n_atoms, (E,), generator=g, dtype=torch.int32)
    c0 = torch.randn(E, N, generator=g)
    got2 = gemm_gather([(d(h), d(src)), (d(eps), None)], d(w), out=d(c0), accumulate=True, row_add=(d(q), d(qi)))
    exact2 = exact + c0.double() + q.double()[qi.long()]
    assert oops.relative(got2.cpu().numpy(), exact2.numpy()) < 1e-5


@pytest.mark.gpu
def test_gemm_split_planes_dynamic_range(device):
    """The three-plane bf16 path must keep fp32 accuracy over a wide exponent range: rows and
    columns scaled by 2^-30 .. 2^30, exact zeros, and values whose low bits the first two planes
    cannot hold (x = 1 + 2^-20). Checked against fp64 row by row (relative to each row's max)."""
    import torch

    from fastmd_amd.ops.wide_gemm import gemm

    g = torch.Generator().manual_seed(13)
    m, k, n = 40000, 264, 512  # >= 512 tiles: the split-plane kernel
    a = torch.randn(m, k, generator=g)
    a *= torch.pow(2.0, torch.randint(-30, 31, (m, 1), generator=g).float())
    a[::7, ::5] = 0.0
    a[1::11] = 1.0 + 2.0 ** -20
    w = torch.randn(n, k, generator=g) / k ** 0.5
    w *= torch.pow(2.0, torch.randint(-8, 9, (n, 1), generator=g).float())
    ref = a.double() @ w.double().t()
    y = gemm(a.to(device), w.to(device), b_layout=0).cpu().double()
    rowmax = ref.abs().max(1, keepdim=True).values.clamp_min(1e-300)
    assert float(((y - ref).abs() / rowmax).max()) < 1e-5


@pytest.mark.gpu
def test_weighted_segment_sum_aggregate_and_count(device):
    """weighted_segment_sum / aggregate / segment_count (the reference's index_add_ and atomic
    variants) against float64 index_add_ on the CPU, on an unsorted segment index with empty
    segments; the weighted form's VJP against float64 autograd."""
    import torch

    from fastmd_amd.ops.segment import aggregate, segment_count, weighted_segment_sum

    g = torch.Generator().manual_seed(21)
    rows, dim, nseg = 5000, 48, 700
    seg = torch.randint(0, nseg - 50, (rows,), generator=g)  # the last 50 segments are empty
    v = torch.randn(rows, dim, generator=g)
    w = torch.randn(rows, dim, generator=g)
    ref = torch.zeros(nseg, dim, dtype=torch.float64).index_add_(0, seg, (w * v).double())
    vd, wd = v.to(device).requires_grad_(), w.to(device).requires_grad_()
    out = weighted_segment_sum(wd, vd, seg.to(device), nseg)
    assert oops.relative(out.detach().cpu().numpy(), ref.numpy()) < 1e-5
    gout = torch.randn(nseg, dim, generator=g)
    out.backward(gout.to(device))
    assert oops.relative(vd.grad.cpu().numpy(), (gout[seg] * w).numpy()) < 1e-6
    assert oops.relative(wd.grad.cpu().numpy(), (gout[seg] * v).numpy()) < 1e-6
    w1 = torch.randn(rows, 1, generator=g)
    out1 = weighted_segment_sum(w1.to(device), v.to(device), seg.to(device), nseg)
    ref1 = torch.zeros(nseg, dim, dtype=torch.float64).index_add_(0, seg, (w1 * v).double())
    assert oops.relative(out1.cpu().numpy(), ref1.numpy()) < 1e-5
    counts = segment_count(seg.to(device), nseg).cpu()
    assert torch.equal(counts, torch.bincount(seg, minlength=nseg))
    mean = aggregate(v.to(device), seg.to(device), num_segment=nseg).cpu().double()
    ref_sum = torch.zeros(nseg, dim, dtype=torch.float64).index_add_(0, seg, v.double())
    ref_mean = ref_sum / counts.clamp_min(1).double()[:, None]
    assert oops.relative(mean.numpy(), ref_mean.numpy()) < 1e-5
    total = aggregate(v.to(device), seg.to(device), average=False).cpu().double()
    assert total.shape[0] == int(seg.max()) + 1
    assert oops.relative(total.numpy(), ref_sum[: total.shape[0]].numpy()) < 1e-5
