"""The node-factored forward message kernel (fmd_mace_message_f32, z_per_node = 1) against a
float64 restatement of its sums on the CPU, on random CSR rows: atoms with no rows, rows longer
than a 64-row chunk, padding rows past the real count, a permuted atom order, C = 64 / 128 / 256,
nb = 8 and 12 (radial rows padded to 16), with and without vector features, one and four waves
per atom. GPU only."""
import numpy as np
import pytest
import torch

from fastmd_amd import _abi


def _rows(n, seed, max_deg=90):
    g = np.random.default_rng(seed)
    deg = g.integers(0, max_deg + 1, size=n)
    deg[g.integers(0, n, size=max(1, n // 17))] = 0  # some atoms without rows
    off = np.zeros(n + 1, dtype=np.int64)
    off[1:] = np.cumsum(deg)
    E = int(off[-1])
    centre = np.repeat(np.arange(n), deg)
    nbr = g.integers(0, n, size=E)
    return g, off, np.stack([centre, nbr], axis=1).astype(np.int32), E


def _case(n, C, nb, h1, seed):
    g, off, ei, E = _rows(n, seed)
    nz = 4 if h1 else 2
    u = g.normal(size=(E, 3))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    geo = np.zeros((E, 8), dtype=np.float32)
    geo[:, :3] = u
    geo[:, 3] = g.uniform(1.0, 6.0, size=E)
    geo[:, 4] = g.uniform(0.0, 1.0, size=E)
    f = lambda *s: (g.normal(size=s) * 0.5).astype(np.float32)
    return dict(off=off, ei=ei, E=E, geo=geo, ef=f(E, nb), P=f(n, nz * C), Q=f(n, nz * C), h0=f(n, C),
                h1=f(n, 3, C) if h1 else None, w1ef=f(nb, 4 * C), n=n, C=C, nb=nb, nz=nz)


def _reference(c, rows):
    """float64: A0[i] = sum_e m0, A1[i] = sum_e m1 over the real rows of each centre."""
    d = lambda a: torch.tensor(a, dtype=torch.float64)
    C, nz = c["C"], c["nz"]
    ei = torch.tensor(c["ei"][:rows].astype(np.int64))
    i, j = ei[:, 0], ei[:, 1]
    geo = d(c["geo"][:rows])
    z = d(c["P"])[j] + d(c["Q"])[i] + d(c["ef"][:rows]) @ d(c["w1ef"])[:, :nz * C]
    w = z * torch.sigmoid(z) * geo[:, 4:5]
    u = geo[:, :3]
    hj = d(c["h0"])[j]
    m0 = w[:, :C] * hj
    m1 = (w[:, C:2 * C] * hj)[:, None, :] * u[:, :, None]
    if c["h1"] is not None:
        hv = d(c["h1"])[j]
        m0 = m0 + w[:, 2 * C:3 * C] * (hv * u[:, :, None]).sum(1)
        m1 = m1 + w[:, None, 3 * C:] * hv
    n = c["n"]
    A0 = torch.zeros(n, C, dtype=torch.float64).index_add_(0, i, m0)
    A1 = torch.zeros(n, 3, C, dtype=torch.float64).index_add_(0, i, m1)
    return A0, A1


def _run(c, device, order, rows, inv_avg, wpa):
    t = lambda a: None if a is None else torch.tensor(a, device=device)
    P, Q, geo, ef, w1ef, h0, h1 = (t(c[k]) for k in ("P", "Q", "geo", "ef", "w1ef", "h0", "h1"))
    ei, off = t(c["ei"]), t(c["off"])
    ne = torch.tensor([rows], dtype=torch.int64, device=device)
    A0 = torch.full((c["n"], c["C"]), float("nan"), device=device)
    A1 = torch.full((c["n"], 3, c["C"]), float("nan"), device=device)
    _abi.call("fmd_mace_message_f32", P.data_ptr(), Q.data_ptr(), geo.data_ptr(), ei.data_ptr(), off.data_ptr(),
              ne.data_ptr(), c["E"], c["n"], _abi.ptr(order), c["C"], h0.data_ptr(), _abi.ptr(h1), inv_avg,
              A0.data_ptr(), A1.data_ptr(), 1, ef.data_ptr(), w1ef.data_ptr(), c["nb"], wpa,
              _abi.stream_handle(device))
    torch.cuda.synchronize()
    return A0.cpu().double(), A1.cpu().double()


@pytest.mark.gpu
@pytest.mark.parametrize("n,C,nb,h1,wpa", [(301, 128, 8, True, 1), (301, 128, 8, False, 1), (157, 64, 8, True, 1),
                                           (157, 256, 8, True, 1), (211, 128, 12, True, 1),
                                           (211, 64, 12, False, 1), (137, 128, 8, True, 4)])
def test_factored_message_matches_float64(device, n, C, nb, h1, wpa):
    print(f"[message] n={n} C={C} nb={nb} h1={h1} wpa={wpa}", flush=True)
    c = _case(n, C, nb, h1, seed=n + C + nb)
    rows = c["E"] - 5  # five padding rows past the real count (not summed)
    inv_avg = 0.125
    perm = torch.tensor(np.random.default_rng(7).permutation(n).astype(np.int32), device=device)
    A0, A1 = _run(c, device, perm, rows, inv_avg, wpa)
    R0, R1 = _reference(c, rows)
    R0, R1 = R0 * inv_avg, R1 * inv_avg
    scale = max(float(R0.abs().max()), float(R1.abs().max()))
    assert float((A0 - R0).abs().max()) <= 2e-6 * scale and float((A1 - R1).abs().max()) <= 2e-6 * scale
    # any atom order gives the same bits, and the same call the same bits again
    B0, B1 = _run(c, device, None, rows, inv_avg, wpa)
    assert torch.equal(A0, B0) and torch.equal(A1, B1)
    D0, D1 = _run(c, device, perm, rows, inv_avg, wpa)
    assert torch.equal(A0, D0) and torch.equal(A1, D1)
