"""(d) The wide edge GEMM on CDNA4 MFMA (HIP kernels).

Reference signatures (fastmd/engine/kernels/triton_wide_gemm.py:482-553):
  ``linear(x, weight, bias=None, precision=None, parts=())`` = ``F.linear`` (y = x W^T + b),
  ``linear_into(out, x, weight, bias=None, rows=None)`` (no autograd),
  ``matmul(grad, weight, c=None, rows=None, accumulate=False, enabled=None)`` = ``grad @ weight (+ c)``.
The reference's 3xTF32 kernels decline K % 16 != 0 (:235), i.e. the configs' K = 2F + 8, and fall
back to cuBLAS SGEMM. Here large K-contiguous ("NT") GEMMs run fp32-accurate on the bf16 matrix
cores (each operand split into three bf16 planes, six MFMA products: CDNA4's counterpart of
3xTF32), the rest on fp32 MFMA (v_mfma_f32_32x32x2_f32); ``edge_gemm(a, w, dtype=torch.bfloat16)``
runs plain bf16 operands (v_mfma_f32_32x32x16_bf16, fp32 out). ``gemm_gather`` fuses the edge-row
gather-cat into the GEMM's operand load. ``epilogue="silu"`` fuses SiLU into the store.
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function

from fastmd_amd import _abi
from fastmd_amd._device import require_cuda, rows_view, stream

_EPILOGUES = {None: 0, "none": 0, "silu": 1}


def gemm(a: Tensor, b: Tensor, *, b_layout: int, bias: Tensor | None = None, out: Tensor | None = None,
         accumulate: bool = False, epilogue: str | None = None) -> Tensor:
    """``a @ op(b) (+ bias) (+ out)``: op(b) = b^T for b_layout 0 (b [N, K]), b for 1 (b [K, N])."""
    require_cuda(a, b, bias, out)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("gemm takes 2-D operands")
    m, k = a.shape
    n = b.shape[0] if b_layout == 0 else b.shape[1]
    kb = b.shape[1] if b_layout == 0 else b.shape[0]
    if kb != k:
        raise ValueError(f"gemm shape mismatch: {tuple(a.shape)} x {tuple(b.shape)} (layout {b_layout})")
    if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float32):
        raise ValueError("bias must be float32 [N]")
    if bias is not None:
        bias = bias.contiguous()
    if out is None:
        out = (torch.zeros if accumulate else torch.empty)((m, n), dtype=torch.float32, device=a.device)
    elif out.shape != (m, n) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [M, N] with unit column stride")
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        name = "fmd_gemm_f32"
    elif a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16:
        name = "fmd_gemm_bf16"
    else:
        raise ValueError(f"gemm operands must both be float32 or bfloat16, got {a.dtype}, {b.dtype}")
    a, lda = rows_view(a)
    b, ldb = rows_view(b)
    if m == 0 or n == 0:
        return out
    _abi.call(name, a.data_ptr(), lda, b.data_ptr(), ldb, b_layout, _abi.ptr(bias), out.data_ptr(),
              out.stride(0) if m > 1 else n, m, n, k, 1 if accumulate else 0, _EPILOGUES[epilogue], stream())
    return out


# 128 x 128 tiles from which a group with pre-split weights takes the split-plane form (below,
# the fp32 kernel's 64 x 64 tiles give four times more workgroups)
GROUP_X3_MIN_TILES = 128
# 64 x 64 tiles below which a b_layout 0 group (and a split-K product) takes the K-split form
# (fmd_gemm_group_ks_f32: 16 x 16 tiles, K shared by the four waves of a workgroup): a group
# that small leaves most of the chip idle while each 64 x 64 tile walks its K slices
GROUP_KS_MAX_TILES = 256


def gemm_group(problems, *, b_layout: int, epilogue: str | None = None) -> list:
    """Up to four independent ``gemm`` problems of one ``b_layout`` in one launch
    (fmd_gemm_group_f32). Each problem is a dict with ``a``, ``b``, ``out`` (float32, preallocated,
    unit column stride) and optionally ``a2`` (extra K columns: ``[a | a2] @ op(b)``, a's width a
    multiple of 32), ``bias``, ``accumulate``, ``row_add`` (``(table, index)``: row ``index[r]`` of the
    float32 ``table`` [*, N] added to output row r, int32 ``index`` [M]; the bits of a prefill of
    those rows and an accumulating launch), and ``b_planes``
    (``split_planes(b)`` of a ``b_layout`` 0 weight): when every problem has them and the group is
    large enough for the split-plane form, the launch reads the planes
    (fmd_gemm_group_x3_planes_rows_f32; the same bits as splitting ``b`` in the kernel, the rows
    added in the epilogue). On the other forms ``row_add`` becomes a prefill of the output
    (fmd_embed_f32) and an accumulating launch: the same bits. Returns the outputs."""
    if not 1 <= len(problems) <= 4:
        raise ValueError("gemm_group takes one to four problems")
    cols = {k: [] for k in ("a", "lda", "a2", "lda2", "ksplit", "b", "ldb", "bias", "c", "ldc", "m", "n", "k", "acc",
                            "radd", "ridx", "rld")}
    keep = []
    for p in problems:
        a, b, out, a2, bias = p["a"], p["b"], p["out"], p.get("a2"), p.get("bias")
        require_cuda(a, b, out, a2, bias)
        for t in (a, b, out) + ((a2,) if a2 is not None else ()):
            if t.dim() != 2 or t.dtype != torch.float32:
                raise ValueError("gemm_group operands must be 2-D float32")
        a, lda = rows_view(a)
        b, ldb = rows_view(b)
        m, ka = a.shape
        k2 = 0
        if a2 is not None:
            a2, lda2 = rows_view(a2)
            if a2.shape[0] != m or ka % 32 != 0:
                raise ValueError("gemm_group: a2 must have a's rows and a's width must be a multiple of 32")
            k2 = a2.shape[1]
        k = ka + k2
        n = b.shape[0] if b_layout == 0 else b.shape[1]
        if (b.shape[1] if b_layout == 0 else b.shape[0]) != k:
            raise ValueError(f"gemm_group shape mismatch: K {k} vs b {tuple(b.shape)} (layout {b_layout})")
        if out.shape != (m, n) or out.stride(1) != 1:
            raise ValueError(f"gemm_group: out must be [{m}, {n}] with unit column stride")
        if bias is not None:
            if bias.shape != (n,) or bias.dtype != torch.float32:
                raise ValueError("bias must be float32 [N]")
            bias = bias.contiguous()
        keep += [a, b, out, a2, bias]
        cols["a"].append(a.data_ptr())
        cols["lda"].append(lda)
        cols["a2"].append(None if a2 is None else a2.data_ptr())
        cols["lda2"].append(0 if a2 is None else lda2)
        cols["ksplit"].append(ka if a2 is not None else k)
        cols["b"].append(b.data_ptr())
        cols["ldb"].append(ldb)
        cols["bias"].append(None if bias is None else bias.data_ptr())
        cols["c"].append(out.data_ptr())
        cols["ldc"].append(out.stride(0) if m > 1 else n)
        cols["m"].append(m)
        cols["n"].append(n)
        cols["k"].append(k)
        cols["acc"].append(1 if p.get("accumulate") else 0)
        ra = p.get("row_add")
        if ra is not None:
            table, index = ra
            require_cuda(table, index)
            if (table.dtype != torch.float32 or table.dim() != 2 or table.shape[1] != n or table.stride(1) != 1
                    or index.dtype != torch.int32 or index.shape != (m,) or not index.is_contiguous()):
                raise ValueError(f"gemm_group: row_add must be a float32 [*, {n}] table and an int32 [{m}] index")
            keep += [table, index]
        cols["radd"].append(None if ra is None else ra[0].data_ptr())
        cols["ridx"].append(None if ra is None else ra[1].data_ptr())
        cols["rld"].append(0 if ra is None else ra[0].stride(0))
    i64 = lambda key: _abi.array(_abi._i64, cols[key])  # noqa: E731

    def prefill_rows() -> None:
        """The forms without the row epilogue: the rows written into the outputs first, then added to."""
        for j, p in enumerate(problems):
            if p.get("row_add") is None:
                continue
            table, index = p["row_add"]
            out = p["out"]
            if p.get("accumulate") or not out.is_contiguous() or not table.is_contiguous():
                raise ValueError("gemm_group: row_add on this form needs a contiguous output and table, no accumulate")
            _abi.call("fmd_embed_f32", index.data_ptr(), table.data_ptr(), out.shape[0], out.shape[1], out.data_ptr(),
                      stream())
            cols["acc"][j] = 1
    planes = [p.get("b_planes") for p in problems]
    tiles64 = sum(-(-m // 64) * -(-n // 64) for m, n in zip(cols["m"], cols["n"]))
    rows_added = any(r is not None for r in cols["radd"])
    if b_layout == 0 and tiles64 < GROUP_KS_MAX_TILES:
        if rows_added:
            prefill_rows()
            rows_added = False
        status = _abi.load().fmd_gemm_group_ks_f32(
            len(problems), _abi.ptr_array(cols["a"]), i64("lda"), _abi.ptr_array(cols["a2"]), i64("lda2"),
            i64("ksplit"), _abi.ptr_array(cols["b"]), i64("ldb"), _abi.ptr_array(cols["bias"]),
            _abi.ptr_array(cols["c"]), i64("ldc"), i64("m"), i64("n"), i64("k"), _abi.array(_abi._i32, cols["acc"]),
            _EPILOGUES[epilogue], stream())
        if status != _EUNSUPPORTED:
            _abi.check(status, "fmd_gemm_group_ks_f32")
            return [p["out"] for p in problems]
    tiles = sum(-(-m // 128) * -(-n // 128) for m, n in zip(cols["m"], cols["n"]))
    if b_layout == 0 and all(q is not None for q in planes) and tiles >= GROUP_X3_MIN_TILES:
        for q, p in zip(planes, problems):
            require_cuda(q.data)
            if q.width != p["b"].shape[1] or q.data.shape[0] != p["b"].shape[0]:
                raise ValueError("gemm_group: b_planes are not the planes of b")
        status = _abi.load().fmd_gemm_group_x3_planes_rows_f32(
            len(problems), _abi.ptr_array(cols["a"]), i64("lda"), _abi.ptr_array(cols["a2"]), i64("lda2"),
            i64("ksplit"), _abi.ptr_array([q.data.data_ptr() for q in planes]),
            _abi.array(_abi._i64, [q.ld for q in planes]), _abi.ptr_array(cols["bias"]), _abi.ptr_array(cols["c"]),
            i64("ldc"), i64("m"), i64("n"), i64("k"), _abi.array(_abi._i32, cols["acc"]),
            _abi.ptr_array(cols["radd"]) if rows_added else None, _abi.ptr_array(cols["ridx"]) if rows_added else None,
            i64("rld") if rows_added else None, _EPILOGUES[epilogue], stream())
        if status != _EUNSUPPORTED:
            _abi.check(status, "fmd_gemm_group_x3_planes_rows_f32")
            return [p["out"] for p in problems]
    if rows_added:
        prefill_rows()
    _abi.call("fmd_gemm_group_f32", len(problems), _abi.ptr_array(cols["a"]), i64("lda"), _abi.ptr_array(cols["a2"]),
              i64("lda2"), i64("ksplit"), _abi.ptr_array(cols["b"]), i64("ldb"), b_layout,
              _abi.ptr_array(cols["bias"]), _abi.ptr_array(cols["c"]), i64("ldc"), i64("m"), i64("n"), i64("k"),
              _abi.array(_abi._i32, cols["acc"]), _EPILOGUES[epilogue], stream())
    return [p["out"] for p in problems]


def gemm_splitk(a: Tensor, b: Tensor, *, b_layout: int, out: Tensor, a2: Tensor | None = None,
                bias: Tensor | None = None, accumulate: bool = False, splits: int = 8,
                b_planes: "Planes | None" = None) -> Tensor:
    """``out (+)= [a | a2] @ op(b) (+ bias)`` with K cut into ``splits`` slices multiplied by separate
    workgroups and summed in slice order (fmd_gemm_splitk_f32): tall-K, few-tile GEMMs. Products
    of fewer than ``GROUP_KS_MAX_TILES`` 64 x 64 tiles (b_layout 0) run as a one-problem K-split
    group instead (one launch, no workspace). With ``b_planes`` (``split_planes(b)``, b_layout 0)
    and a large enough product: four (or two) K slices as split-plane problems of one grouped
    launch, summed in order (fmd_gemm_splitk_x3_planes_f32)."""
    require_cuda(a, b, out, a2, bias)
    n_out = b.shape[0] if b_layout == 0 else b.shape[1]
    if b_planes is not None and b_layout == 0 and -(-a.shape[0] // 64) * -(-n_out // 64) >= GROUP_KS_MAX_TILES:
        done = _splitk_planes(a, b_planes, out, a2, bias, accumulate)
        if done:
            return out
    if b_layout == 0 and -(-a.shape[0] // 64) * -(-n_out // 64) < GROUP_KS_MAX_TILES and (
            a2 is None or a.shape[1] % 32 == 0):
        prob = {"a": a, "b": b, "out": out, "accumulate": accumulate}
        if a2 is not None:
            prob["a2"] = a2
        if bias is not None:
            prob["bias"] = bias
        gemm_group([prob], b_layout=0)
        return out
    a, lda = rows_view(a)
    b, ldb = rows_view(b)
    m, ka = a.shape
    k = ka + (a2.shape[1] if a2 is not None else 0)
    n = b.shape[0] if b_layout == 0 else b.shape[1]
    if (b.shape[1] if b_layout == 0 else b.shape[0]) != k or out.shape != (m, n) or out.stride(1) != 1:
        raise ValueError("gemm_splitk shape mismatch")
    lda2 = 0
    if a2 is not None:
        a2, lda2 = rows_view(a2)
        if a2.shape[0] != m:
            raise ValueError("gemm_splitk: a2 must have a's rows")
    while splits > 1 and (k % splits or (k // splits) % 32 or (a2 is not None and ka % (k // splits))):
        splits //= 2
    ws = torch.empty((splits, m, n), dtype=torch.float32, device=out.device)
    if bias is not None:
        bias = bias.contiguous()
    _abi.call("fmd_gemm_splitk_f32", a.data_ptr(), lda, _abi.ptr(a2), lda2, ka, b.data_ptr(), ldb, b_layout,
              _abi.ptr(bias), out.data_ptr(), out.stride(0) if m > 1 else n, m, n, k, 1 if accumulate else 0, splits,
              ws.data_ptr(), stream())
    return out


def _splitk_planes(a, planes, out, a2, bias, accumulate) -> bool:
    """fmd_gemm_splitk_x3_planes_f32 when the layout allows it (else False, nothing launched)."""
    a, lda = rows_view(a)
    m, ka = a.shape
    k = ka + (a2.shape[1] if a2 is not None else 0)
    n = out.shape[1]
    if planes.width != k or planes.data.shape[0] != n or out.shape[0] != m or out.stride(1) != 1:
        raise ValueError("gemm_splitk: b_planes do not match")
    lda2 = 0
    if a2 is not None:
        a2, lda2 = rows_view(a2)
    splits = next((s for s in (4, 2) if k % s == 0 and (k // s) % 16 == 0 and ka % (k // s) == 0), 0)
    ok = (splits and lda % 4 == 0 and a.data_ptr() % 16 == 0 and
          (a2 is None or (lda2 % 4 == 0 and a2.data_ptr() % 16 == 0)))
    if not ok:
        return False
    ws = torch.empty((splits, m, n), dtype=torch.float32, device=out.device)
    if bias is not None:
        bias = bias.contiguous()
    _abi.call("fmd_gemm_splitk_x3_planes_f32", a.data_ptr(), lda, _abi.ptr(a2), lda2, ka, planes.data.data_ptr(),
              48 * planes.data.shape[1], _abi.ptr(bias), out.data_ptr(), out.stride(0) if m > 1 else n, m, n, k,
              1 if accumulate else 0, splits, ws.data_ptr(), stream())
    return True


class Planes:
    """The three bf16 planes of a float32 matrix [rows, width] (fmd_split3_f32), slice-interleaved:
    ``data`` [rows, S, 3, 16] bfloat16 (S = ceil(width / 16), zero past ``width``), x = p0 + p1 + p2."""

    __slots__ = ("data", "width")

    def __init__(self, data: Tensor, width: int) -> None:
        self.data, self.width = data, int(width)

    @property
    def ld(self) -> int:
        """Row stride in elements (48 S)."""
        return self.data.shape[1] * 48

    def dense(self) -> Tensor:
        """[rows, 3, 16 S] view order of the planes (a copy), for checks."""
        rows, slices = self.data.shape[:2]
        return self.data.permute(0, 2, 1, 3).reshape(rows, 3, slices * 16)


def split_planes(x: Tensor, *, out: Planes | None = None) -> Planes:
    """The bf16 planes of a 2-D float32 ``x`` (fmd_split3_f32)."""
    require_cuda(x)
    if x.dim() != 2 or x.dtype != torch.float32:
        raise ValueError("split_planes takes a 2-D float32 tensor")
    x, ld = rows_view(x)
    rows, width = x.shape
    slices = -(-width // 16)
    if out is None:
        out = Planes(torch.empty((rows, slices, 3, 16), dtype=torch.bfloat16, device=x.device), width)
    elif out.data.shape != (rows, slices, 3, 16) or out.width != width:
        raise ValueError("split_planes: out does not match")
    if rows:
        _abi.call("fmd_split3_f32", x.data_ptr(), ld, rows, width, out.data.data_ptr(), stream())
    return out


def gemm_planes(parts, b: Planes, *, a_planes: bool, out: Tensor | None = None, bias: Tensor | None = None,
                accumulate: bool = False, epilogue: str | None = None, row_add=None) -> Tensor:
    """``gemm_gather`` with pre-split operands (fmd_gemm_x3_planes_f32): ``b`` the planes of the
    K-contiguous weight [N, K] (``split_planes(w)``), ``parts`` a list of up to three
    ``(src, index)`` with ``src`` Planes (``a_planes``) or float32 [rows, width]. Bitwise equal to
    ``gemm_gather`` on the unsplit operands."""
    if not 1 <= len(parts) <= 3:
        raise ValueError("gemm_planes takes one to three parts")
    require_cuda(b.data, out, bias)
    rows = None
    srcs, idx, strides, lds, widths, keep = [], [], [], [], [], []
    for src, index in parts:
        if a_planes:
            if not isinstance(src, Planes):
                raise ValueError("gemm_planes(a_planes=True) takes Planes parts")
            data, ld, width, n_src = src.data, src.ld, src.width, src.data.shape[0]
        else:
            if src.dtype != torch.float32 or src.dim() != 2:
                raise ValueError("gemm_planes parts must be 2-D float32")
            data, ld = rows_view(src)
            width, n_src = data.shape[1], data.shape[0]
        require_cuda(data)
        if index is not None:
            if index.dtype != torch.int32 or index.dim() != 1:
                index = index.to(torch.int32).reshape(-1).contiguous()
            n_rows = index.numel()
            stride = index.stride(0) if n_rows > 1 else 1
        else:
            n_rows, stride = n_src, 1
        if rows is None:
            rows = n_rows
        elif n_rows != rows:
            raise ValueError("gemm_planes parts disagree on the row count")
        keep += [data, index]
        srcs.append(data.data_ptr())
        idx.append(None if index is None else index.data_ptr())
        strides.append(stride)
        lds.append(ld)
        widths.append(width)
    k = sum(widths)
    if b.width != k:
        raise ValueError(f"gemm_planes: b has K = {b.width}, the parts {k}")
    n = b.data.shape[0]
    if bias is not None:
        if bias.shape != (n,) or bias.dtype != torch.float32:
            raise ValueError("bias must be float32 [N]")
        bias = bias.contiguous()
    if out is None:
        out = (torch.zeros if accumulate else torch.empty)((rows, n), dtype=torch.float32, device=b.data.device)
    elif out.shape != (rows, n) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [M, N] with unit column stride")
    q, qidx, qstride, ldq = None, None, 1, 0
    if row_add is not None:
        q, qidx = row_add
        if q.dim() != 2 or q.dtype != torch.float32 or q.shape[1] != n or q.stride(1) != 1:
            raise ValueError(f"row_add must be float32 [*, {n}] with unit column stride")
        ldq = q.stride(0)
        if qidx is not None:
            qstride = qidx.stride(0) if rows > 1 else 1
    if rows == 0 or n == 0:
        return out
    _abi.call("fmd_gemm_x3_planes_f32", 1 if a_planes else 0, len(parts), _abi.ptr_array(srcs), _abi.ptr_array(idx),
              _abi.array(_abi._i64, strides), _abi.array(_abi._i64, lds), _abi.array(_abi._i32, widths), rows,
              b.data.data_ptr(), b.ld, k, _abi.ptr(q), _abi.ptr(qidx), qstride, ldq, _abi.ptr(bias), out.data_ptr(),
              out.stride(0) if rows > 1 else n, n, 1 if accumulate else 0, _EPILOGUES[epilogue], stream())
    return out


_EUNSUPPORTED = 10002


def gemm_gather(parts, b: Tensor, *, out: Tensor | None = None, bias: Tensor | None = None,
                accumulate: bool = False, epilogue: str | None = None, row_add=None) -> Tensor:
    """``cat([src[idx] or src for src, idx in parts], 1) @ b^T (+ q[qidx])`` with the gather-cat
    fused into the GEMM's operand load (fmd_gemm_gather_f32): ``parts`` is a list of up to three
    ``(src, index)`` (``index`` None: row r of ``src``; an int32 index may be a strided column
    view), ``b`` [N, K] K-contiguous, ``row_add`` an optional ``(q [*, N], qidx or None)`` whose
    gathered row is added to each output row. Falls back to gather-cat + GEMM (+ add) when the
    layout does not meet the fused kernel's conditions (16-byte aligned rows, widths % 4, all but
    the last width % 16)."""
    require_cuda(b, out, bias, *[src for src, _ in parts])
    if not 1 <= len(parts) <= 3:
        raise ValueError("gemm_gather takes one to three parts")
    rows = None
    srcs, idx, strides, lds, widths, keep = [], [], [], [], [], []
    for src, index in parts:
        if src.dtype != torch.float32 or src.dim() != 2:
            raise ValueError("gemm_gather parts must be 2-D float32")
        src, ld = rows_view(src)
        if index is not None:
            if index.dtype != torch.int32 or index.dim() != 1:
                index = index.to(torch.int32).reshape(-1).contiguous()
            n_rows = index.numel()
            stride = index.stride(0) if n_rows > 1 else 1
        else:
            n_rows, stride = src.shape[0], 1
        if rows is None:
            rows = n_rows
        elif n_rows != rows:
            raise ValueError("gemm_gather parts disagree on the row count")
        keep += [src, index]
        srcs.append(src.data_ptr())
        idx.append(None if index is None else index.data_ptr())
        strides.append(stride)
        lds.append(ld)
        widths.append(src.shape[1])
    k = sum(widths)
    if b.dim() != 2 or b.dtype != torch.float32 or b.shape[1] != k or b.stride(1) != 1:
        raise ValueError(f"gemm_gather: b must be float32 [N, {k}] with unit column stride")
    n = b.shape[0]
    if bias is not None and (bias.shape != (n,) or bias.dtype != torch.float32):
        raise ValueError("bias must be float32 [N]")
    if bias is not None:
        bias = bias.contiguous()
    if out is None:
        out = (torch.zeros if accumulate else torch.empty)((rows, n), dtype=torch.float32, device=b.device)
    elif out.shape != (rows, n) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError("out must be float32 [M, N] with unit column stride")
    q, qidx, qstride, ldq = None, None, 1, 0
    if row_add is not None:
        q, qidx = row_add
        require_cuda(q, qidx)
        if q.dim() != 2 or q.dtype != torch.float32 or q.shape[1] != n or q.stride(1) != 1:
            raise ValueError(f"row_add must be float32 [*, {n}] with unit column stride")
        ldq = q.stride(0)
        if qidx is not None:
            if qidx.dtype != torch.int32 or qidx.dim() != 1 or qidx.numel() != rows:
                raise ValueError(f"row_add index must be int32 [{rows}]")
            qstride = qidx.stride(0) if rows > 1 else 1
        elif q.shape[0] != rows:
            raise ValueError(f"row_add without an index needs {rows} rows")
    if rows == 0 or n == 0:
        return out
    status = _abi.load().fmd_gemm_gather_f32(
        len(parts), _abi.ptr_array(srcs), _abi.ptr_array(idx), _abi.array(_abi._i64, strides),
        _abi.array(_abi._i64, lds), _abi.array(_abi._i32, widths), rows, b.data_ptr(), b.stride(0),
        _abi.ptr(q), _abi.ptr(qidx), qstride, ldq, _abi.ptr(bias), out.data_ptr(),
        out.stride(0) if rows > 1 else n, n, 1 if accumulate else 0, _EPILOGUES[epilogue], stream())
    if status == _EUNSUPPORTED:
        from fastmd_amd.ops.gather_cat import _launch as gather_launch

        if row_add is not None and (bias is not None or accumulate or epilogue not in (None, "none")):
            raise ValueError("gemm_gather fallback: row_add with bias/accumulate/epilogue is not supported")
        a = torch.empty((rows, k), dtype=torch.float32, device=b.device)
        gather_launch(parts, rows, a)
        gemm(a, b, b_layout=0, bias=bias, out=out, accumulate=accumulate, epilogue=epilogue)
        if row_add is not None:
            out += q if qidx is None else q.index_select(0, qidx.long())
        return out
    _abi.check(status, "fmd_gemm_gather_f32")
    return out


class _Linear(Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        y = gemm(x, weight, b_layout=0, bias=bias)
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight = ctx.saved_tensors
        gy = gy.contiguous()
        gx = gemm(gy, weight, b_layout=1) if ctx.needs_input_grad[0] else None
        # trainable weights are outside the MD path (the reference declines them too,
        # triton_wide_gemm.py:242-243): their gradient is formed by torch
        gw = gy.t().mm(x) if ctx.needs_input_grad[1] else None
        gb = gy.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb


def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, precision=None, parts=()) -> Tensor:
    """``F.linear(x, weight, bias)`` on the MFMA kernels (x 2-D float32). ``precision`` and
    ``parts`` are accepted for signature parity; there is one precision, fp32-accurate (fp32
    MFMA, or three bf16 planes per operand for the large K-contiguous shapes)."""
    if x.dim() != 2:
        shape = x.shape
        return linear(x.reshape(-1, shape[-1]), weight, bias).reshape(*shape[:-1], weight.shape[0])
    return _Linear.apply(x, weight, bias)


def linear_into(out: Tensor, x: Tensor, weight: Tensor, bias: Tensor | None = None, rows: int | None = None):
    """``out[:] = x @ weight^T (+ bias)`` (no autograd); ``rows`` is accepted for parity (a row chunk
    takes the same kernel as the whole GEMM, so the rows are equal either way)."""
    with torch.no_grad():
        return gemm(x, weight, b_layout=0, bias=bias, out=out)


def matmul(grad: Tensor, weight: Tensor, c: Tensor | None = None, rows: int | None = None, accumulate: bool = False,
           enabled: bool | None = None) -> Tensor:
    """``grad @ weight (+ c)``; ``accumulate`` writes into ``c``."""
    with torch.no_grad():
        if c is None:
            return gemm(grad, weight, b_layout=1)
        if accumulate:
            return gemm(grad, weight, b_layout=1, out=c, accumulate=True)
        out = c.clone()
        return gemm(grad, weight, b_layout=1, out=out, accumulate=True)


def edge_gemm(a: Tensor, w: Tensor, dtype: torch.dtype = torch.float32, *, bias: Tensor | None = None,
              epilogue: str | None = None) -> Tensor:
    """The configs' wide edge GEMM ``[E, 2F+8] x [2F+8, 4F]`` with ``w`` stored ``[2F+8, 4F]``
    (b_layout 1); ``dtype`` float32 or bfloat16 operands, float32 output. No autograd."""
    with torch.no_grad():
        if dtype == torch.bfloat16:
            # the weight transposed once to K-contiguous [4F, 2F+8]: the direct-to-LDS bf16 kernel
            return gemm(a.to(torch.bfloat16), w.t().contiguous().to(torch.bfloat16), b_layout=0, bias=bias,
                        epilogue=epilogue)
        if dtype != torch.float32:
            raise ValueError(f"edge_gemm dtype must be float32 or bfloat16, got {dtype}")
        # the weight transposed once to K-contiguous [4F, 2F+8]: the layout of the fp32-accurate
        # split-plane kernel
        return gemm(a, w.t().contiguous(), b_layout=0, bias=bias, epilogue=epilogue)
