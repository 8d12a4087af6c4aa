"""SVD-MLP operators on MI355X: the kernels/reference.py API backed by HIP.

    fused_gate_up(x, u_gate, v_gate, u_up, v_up)      kernels/reference.py:54-72
    fused_xuv(x, u, v)                                kernels/reference.py:75-82
    svd_mlp(x, ug, vg, uu, vu, ud, vd)                kernels/reference.py:85-93

Arguments are CUDA (ROCm) tensors.  Factors use the reference's natural
layout, ``u`` (d_in, r) and ``v`` (r, d_out); a factor that is the transpose
view of a contiguous PyTorch ``Linear.weight`` (out, in) is passed to the
kernels without a copy (layout flag).  Activations and factors are bfloat16
or float32 (all the same dtype), or factors are :class:`QuantizedFactor`
(fp8 e4m3fn + per-output-column fp32 scale) with bfloat16 activations.

Every call goes to libsvdmlp.so; there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict
from dataclasses import dataclass

import torch

from . import _lib

_ACT_CODES = {torch.bfloat16: _lib.SVDMLP_BF16, torch.float32: _lib.SVDMLP_F32}


@dataclass(frozen=True)
class QuantizedFactor:
    """An fp8 e4m3fn factor in natural (d_in, d_out) layout with one fp32
    scale per output column: ``w ~= data.float() * scale``."""

    data: torch.Tensor  # (d_in, d_out), torch.float8_e4m3fn (or raw uint8 bits)
    scale: torch.Tensor  # (d_out,), float32

    @property
    def shape(self) -> torch.Size:
        return self.data.shape

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def device(self):
        return self.data.device

    def dim(self) -> int:
        return self.data.dim()

    def dequantize(self) -> torch.Tensor:
        return self.data.view(torch.float8_e4m3fn).float() * self.scale.float()


# ---------------------------------------------------------------------------
# Validation (messages follow test_speedup.py:37-49,508-509,530-533)
# ---------------------------------------------------------------------------

def _shape(a) -> tuple[int, ...]:
    return tuple(a.shape)


def validate_arrays(*arrays) -> None:
    """Reference ``_validate_arrays`` contract (test_speedup.py:42-49)."""
    for a in arrays:
        if a.dim() != 2 or min(_shape(a)) <= 0:
            raise ValueError(f"expected a nonempty 2D array, got {_shape(a)}")
    quant = [isinstance(a, QuantizedFactor) for a in arrays[1:]]
    if any(quant):
        if not all(quant):
            raise TypeError("all inputs must have the same dtype")
        if arrays[0].dtype != torch.bfloat16:
            raise TypeError("fp8 factors require bfloat16 activations")
        return
    for a in arrays:
        if a.dtype != arrays[0].dtype:
            raise TypeError("all inputs must have the same dtype")
    if arrays[0].dtype not in _ACT_CODES:
        raise TypeError("supported dtypes are bfloat16 and float32")


def _check_device(*tensors) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"SVD-MLP kernels run on a ROCm GPU; got tensors on {dev}")
    for t in tensors:
        if t.device != dev:
            raise ValueError("all inputs must be on the same device")
    return dev


class _Factor:
    """A factor prepared for the C ABI: keeps the tensor alive, records the
    layout (natural or Linear), the row pitch of a row-padded natural-layout
    view (``ld``, elements; 0 when dense) and the fp8 scale."""

    __slots__ = ("tensor", "ptr", "linear", "scale", "scale_ptr", "rows", "cols", "ld")

    def __init__(self, f):
        if isinstance(f, QuantizedFactor):
            data = f.data
            if not data.is_contiguous():
                data = data.contiguous()
            scale = f.scale.to(torch.float32).contiguous()
            if scale.dim() != 1 or scale.numel() != data.shape[1] or scale.device != data.device:
                raise ValueError("fp8 factor scale must hold one value per output column")
            self.tensor, self.linear = data, False
            self.scale, self.scale_ptr = scale, scale.data_ptr()
        else:
            t = f
            linear = False
            self.ld = 0
            if not t.is_contiguous():
                if t.t().is_contiguous():
                    linear = True
                elif padded_rows(t):
                    self.ld = int(t.stride(0))
                else:
                    t = t.contiguous()
            self.tensor, self.linear = t, linear
            self.scale, self.scale_ptr = None, None
        if isinstance(f, QuantizedFactor):
            self.ld = 0
        self.ptr = self.tensor.data_ptr()
        self.rows, self.cols = int(f.shape[0]), int(f.shape[1])

    def dense(self) -> None:
        """Replace a row-padded view by a contiguous copy."""
        if self.ld:
            self.tensor, self.ld = self.tensor.contiguous(), 0
            self.ptr = self.tensor.data_ptr()


def padded_rows(t: torch.Tensor) -> bool:
    """A natural-layout bf16 view whose rows are spaced wider than their
    length (a column slice of a wider buffer), 16-byte aligned rows: the
    layered entry points read it in place."""
    return (t.dim() == 2 and t.dtype == torch.bfloat16 and t.stride(1) == 1 and t.stride(0) > t.shape[1]
            and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0)


def pad_rows(t: torch.Tensor, pad: int = 64) -> torch.Tensor:
    """A copy of the 2-D tensor t whose rows are ``pad`` elements longer in
    memory, returned as the (rows, cols) view: the row pitch that spreads a
    factor's column stripes over all HBM channels (rows of 4096 or 14336
    bf16 elements otherwise map each stripe onto a subset)."""
    rows, cols = t.shape
    buf = torch.zeros((rows, cols + pad), dtype=t.dtype, device=t.device)
    buf[:, :cols] = t
    return buf[:, :cols]


def _w_code(x: torch.Tensor, factors) -> int:
    if isinstance(factors[0], QuantizedFactor):
        return _lib.SVDMLP_FP8_E4M3
    return _ACT_CODES[x.dtype]


def _activation(x: torch.Tensor) -> torch.Tensor:
    return x if x.is_contiguous() else x.contiguous()


def _layout_flags(us, vs) -> int:
    """One layout flag per factor kind; mixed layouts are made uniform."""
    flags = 0
    if all(f.linear for f in us):
        flags |= _lib.SVDMLP_U_LINEAR
    if all(f.linear for f in vs):
        flags |= _lib.SVDMLP_V_LINEAR
    return flags


def _uniform(factors, linear: bool) -> None:
    for f in factors:
        if f.linear != linear:
            # A mix of layouts: give the odd one out the uniform layout.
            # f.tensor is always the logical (d_in, d_out) view.
            f.tensor = f.tensor.t().contiguous().t() if linear else f.tensor.contiguous()
            f.linear, f.ld = linear, 0
            f.ptr = f.tensor.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _workspace(dev, T, d, ff, r, w_code) -> torch.Tensor:
    """Workspace of the C ABI's size; its first 4 KB (grid-barrier words of
    the persistent decode kernel) start at zero, as the ABI requires."""
    nbytes = _lib.workspace_bytes(T, d, ff, r, w_code)
    ws = torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=dev)
    ws[:4096].zero_()
    return ws


# Workspaces of calls that pass none, one per (device, stream), grown on
# demand: every call leaves the first 4 KB valid for the next call on its
# stream (the barrier counters only grow, the tile counters return to zero),
# so a reused workspace needs no clearing; a fresh one per call cost an
# allocation and a fill kernel each time.
_WS_CACHE: dict = {}


_WS_BYTES: dict = {}


def _shared_workspace(dev, T, d, ff, r, w_code) -> torch.Tensor:
    size_key = (T, d, ff, r, w_code)
    nbytes = _WS_BYTES.get(size_key)
    if nbytes is None:
        if len(_WS_BYTES) > 4096:
            _WS_BYTES.clear()
        nbytes = _WS_BYTES[size_key] = max(_lib.workspace_bytes(T, d, ff, r, w_code), 4096)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), torch.cuda.current_stream(dev).cuda_stream)
    ws = _WS_CACHE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        ws[:4096].zero_()
        _WS_CACHE[key] = ws
    return ws


def clear_workspace_cache() -> None:
    """Release the workspaces kept for calls that pass none (allocated again
    on the next such call)."""
    _WS_CACHE.clear()


# ---------------------------------------------------------------------------
# Operators
# ---------------------------------------------------------------------------

def fused_gate_up(x, u_gate, v_gate, u_up, v_up, *, out_transposed: bool = False) -> torch.Tensor:
    """Returns (S, I) = silu(X @ Ug @ Vg) * (X @ Uu @ Vu) in x.dtype
    (kernels/reference.py:54-72); (I, S) when ``out_transposed``."""
    validate_arrays(x, u_gate, v_gate, u_up, v_up)
    T, d = _shape(x)
    if u_gate.shape[0] != d or v_gate.shape[0] != u_gate.shape[1]:
        raise ValueError("X, U, V contraction dimensions do not match")
    if _shape(u_up) != _shape(u_gate) or _shape(v_up) != _shape(v_gate):
        raise ValueError("gate/up factors must have matching shapes")
    r, ff = _shape(v_gate)
    dev = _check_device(x, u_gate, v_gate, u_up, v_up)
    lib = _lib.load()
    x = _activation(x)
    ug, vg, uu, vu = (_Factor(f) for f in (u_gate, v_gate, u_up, v_up))
    for f in (ug, vg, uu, vu):
        f.dense()  # this entry point takes dense rows
    _uniform((ug, uu), ug.linear and uu.linear)
    _uniform((vg, vu), vg.linear and vu.linear)
    flags = _layout_flags((ug, uu), (vg, vu)) | (_lib.SVDMLP_OUT_T if out_transposed else 0)
    w_code = _w_code(x, (u_gate,))
    out = torch.empty((ff, T) if out_transposed else (T, ff), dtype=x.dtype, device=dev)
    ws = _shared_workspace(dev, T, d, ff, r, w_code)
    with torch.cuda.device(dev):
        _lib.check(lib.svdmlp_gate_up(
            x.data_ptr(), ug.ptr, vg.ptr, uu.ptr, vu.ptr,
            ug.scale_ptr, vg.scale_ptr, uu.scale_ptr, vu.scale_ptr,
            out.data_ptr(), T, d, ff, r, _ACT_CODES[x.dtype], w_code, flags,
            ws.data_ptr(), ws.numel(), _stream(dev)))
    return out


def fused_xuv(x, u, v, *, x_transposed: bool = False) -> torch.Tensor:
    """Returns (S, H) = X @ U @ V in x.dtype (kernels/reference.py:75-82).
    With ``x_transposed`` the input is given as X^T, shape (I, S)."""
    validate_arrays(x, u, v)
    if x_transposed:
        din, T = _shape(x)
    else:
        T, din = _shape(x)
    if u.shape[0] != din or v.shape[0] != u.shape[1]:
        raise ValueError("X, U, V contraction dimensions do not match")
    r, dout = _shape(v)
    dev = _check_device(x, u, v)
    lib = _lib.load()
    x = _activation(x)
    fu, fv = _Factor(u), _Factor(v)
    fu.dense()
    fv.dense()
    flags = _layout_flags((fu,), (fv,)) | (_lib.SVDMLP_X_T if x_transposed else 0)
    w_code = _w_code(x, (u,))
    out = torch.empty((T, dout), dtype=x.dtype, device=dev)
    ws = _shared_workspace(dev, T, din, dout, r, w_code)
    with torch.cuda.device(dev):
        _lib.check(lib.svdmlp_xuv(
            x.data_ptr(), fu.ptr, fv.ptr, fu.scale_ptr, fv.scale_ptr, out.data_ptr(),
            T, din, dout, r, _ACT_CODES[x.dtype], w_code, flags,
            ws.data_ptr(), ws.numel(), _stream(dev)))
    return out


# Prepared arguments of layers seen before, keyed on x's dtype, device and
# width and on every factor's address, shape, strides, dtype and device: a
# layer called again skips validation and marshalling (~20 us of Python per
# call, which a lone call's first kernel waits for).  Only layers whose
# factors are all read in place are kept, as addresses: a key can only match
# tensors that lie exactly where the cached pointers point.
_PLANS: dict = {}


def _plan_key(x, factors):
    if type(x) is not torch.Tensor or x.dim() != 2 or x.shape[0] == 0:
        return None
    key = [x.dtype, x.device, x.shape[1]]
    for f in factors:
        if type(f) is not torch.Tensor:
            return None
        key += (f.data_ptr(), f.shape, f.stride(), f.dtype, f.device)
    return tuple(key)


def _prepare_layer(x, u_gate, v_gate, u_up, v_up, u_down, v_down, workspace, out):
    """Validation and argument marshalling shared by svd_mlp and svd_mlp_block;
    returns (x, factor pointers, holders, flags, w_code, scale array, ld
    array, out, workspace, dims, device).  The caller keeps `holders` (the
    prepared factors, which may own contiguous copies) until the launch is
    enqueued."""
    factors = (u_gate, v_gate, u_up, v_up, u_down, v_down)
    key = _plan_key(x, factors)
    plan = _PLANS.get(key) if key is not None else None
    if plan is not None:
        ptrs, flags, w_code, ld_arr, (d, ff, r_g, r_u, r_d), dev = plan
        T = int(x.shape[0])
        x = _activation(x)
        if out is None:
            out = torch.empty((T, d), dtype=x.dtype, device=dev)
        elif out.shape != (T, d) or out.dtype != x.dtype or not out.is_contiguous() or out.device != dev:
            raise ValueError("out must be a contiguous (T, d) tensor of x.dtype on x.device")
        if workspace is None:
            workspace = _shared_workspace(dev, T, d, ff, max(r_g, r_u, r_d), w_code)
        return x, ptrs, None, flags, w_code, None, ld_arr, out, workspace, (T, d, ff, r_g, r_u, r_d), dev
    validate_arrays(x, u_gate, v_gate, u_up, v_up, u_down, v_down)
    T, d = _shape(x)
    if u_gate.shape[0] != d or v_gate.shape[0] != u_gate.shape[1] or v_up.shape[0] != u_up.shape[1]:
        raise ValueError("X, U, V contraction dimensions do not match")
    # the gate and up ranks may differ (kernels/reference.py:54-72 allows it)
    if u_up.shape[0] != u_gate.shape[0] or v_up.shape[1] != v_gate.shape[1]:
        raise ValueError("gate/up factors must have matching shapes")
    r_g, ff = _shape(v_gate)
    r_u = int(v_up.shape[0])
    if u_down.shape[0] != ff or v_down.shape[0] != u_down.shape[1] or v_down.shape[1] != d:
        raise ValueError("X, U, V contraction dimensions do not match")
    r_d = int(u_down.shape[1])
    dev = _check_device(x, u_gate, v_gate, u_up, v_up, u_down, v_down)
    x = _activation(x)
    fs = [_Factor(f) for f in (u_gate, v_gate, u_up, v_up, u_down, v_down)]
    us, vs = (fs[0], fs[2], fs[4]), (fs[1], fs[3], fs[5])
    _uniform(us, all(f.linear for f in us))
    _uniform(vs, all(f.linear for f in vs))
    flags = _layout_flags(us, vs)
    w_code = _w_code(x, (u_gate,))
    # padded rows: bf16 natural layout only, one pitch for gate and up when
    # their ranks are equal (the decode kernels read both with one pitch)
    if x.dtype != torch.bfloat16 or w_code == _lib.SVDMLP_FP8_E4M3 or flags:
        for f in fs:
            f.dense()
    if r_g == r_u:
        for a, b in ((fs[0], fs[2]), (fs[1], fs[3])):
            if a.ld != b.ld:
                a.dense()
                b.dense()
    ld_arr = (ctypes.c_int64 * 6)(*[f.ld for f in fs]) if any(f.ld for f in fs) else None
    scale_arr = None
    if w_code == _lib.SVDMLP_FP8_E4M3:
        scale_arr = (ctypes.c_void_p * 6)(*[f.scale_ptr for f in fs])
    if out is None:
        out = torch.empty((T, d), dtype=x.dtype, device=dev)
    elif out.shape != (T, d) or out.dtype != x.dtype or not out.is_contiguous() or out.device != dev:
        raise ValueError("out must be a contiguous (T, d) tensor of x.dtype on x.device")
    if workspace is None:
        workspace = _shared_workspace(dev, T, d, ff, max(r_g, r_u, r_d), w_code)
    dims = (T, d, ff, r_g, r_u, r_d)
    ptrs = tuple(f.ptr for f in fs)
    if key is not None and scale_arr is None and all(p == f.data_ptr() for p, f in zip(ptrs, factors)):
        if len(_PLANS) > 64:
            _PLANS.clear()
        _PLANS[key] = (ptrs, flags, w_code, ld_arr, (d, ff, r_g, r_u, r_d), dev)
    return x, ptrs, fs, flags, w_code, scale_arr, ld_arr, out, workspace, dims, dev


def _on_device(dev, call):
    """Run call with dev current (a no-op switch when it already is)."""
    if dev.index is None or dev.index == torch.cuda.current_device():
        return call()
    with torch.cuda.device(dev):
        return call()


def pad_rank(u, v, r: int):
    """U (d_in, r0) and V (r0, d_out) zero-padded to rank r: r - r0 more U
    columns and V rows of zeros, which add exactly nothing to U . V.  fp8
    factors pad their data with zeros (and the U scales with ones)."""
    r0 = int(u.shape[1])
    if r0 == r:
        return u, v
    if isinstance(u, QuantizedFactor):
        ud = torch.zeros((u.shape[0], r), dtype=u.data.dtype, device=u.device)
        ud[:, :r0] = u.data
        us = torch.ones(r, dtype=torch.float32, device=u.device)
        us[:r0] = u.scale
        vd = torch.zeros((r, v.shape[1]), dtype=v.data.dtype, device=v.device)
        vd[:r0] = v.data
        return QuantizedFactor(ud, us), QuantizedFactor(vd, v.scale)
    up = torch.zeros((u.shape[0], r), dtype=u.dtype, device=u.device)
    vp = torch.zeros((r, v.shape[1]), dtype=v.dtype, device=v.device)
    up[:, :r0] = u
    vp[:r0] = v
    return up, vp


# Zero-padded gate/up factors of the shapes whose kernels take one rank (the
# SVDMLP_EUNSUP fallback), kept for the most recent layers: keyed by each
# factor's storage address, version counter (bumped by in-place writes),
# shape and dtype, so a layer called again reuses its padded copies instead
# of allocating and copying them on every call.
_PAD_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_PAD_CACHE_LAYERS = 8


def _factor_key(f):
    t = f.data if isinstance(f, QuantizedFactor) else f
    k = (t.data_ptr(), t._version, tuple(t.shape), str(t.dtype))
    if isinstance(f, QuantizedFactor):
        k += (f.scale.data_ptr(), f.scale._version)
    return k


def _pad_branches(u_gate, v_gate, u_up, v_up):
    r = max(int(u_gate.shape[1]), int(u_up.shape[1]))
    key = tuple(_factor_key(f) for f in (u_gate, v_gate, u_up, v_up))
    hit = _PAD_CACHE.get(key)
    if hit is not None:
        _PAD_CACHE.move_to_end(key)
        return hit[1]
    padded = (*pad_rank(u_gate, v_gate, r), *pad_rank(u_up, v_up, r))
    # the originals are held too, so that their addresses are not reused while the entry lives
    _PAD_CACHE[key] = ((u_gate, v_gate, u_up, v_up), padded)
    while len(_PAD_CACHE) > _PAD_CACHE_LAYERS:
        _PAD_CACHE.popitem(last=False)
    return padded


def svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down, *, workspace: torch.Tensor | None = None,
            out: torch.Tensor | None = None, contracted: bool = False,
            fp8_activations: bool = False) -> torch.Tensor:
    """Full SVD SwiGLU block, fused_xuv(fused_gate_up(x)) with h rounded to
    x.dtype in between (kernels/reference.py:85-93).  The gate, up and down
    ranks may all differ: the persistent decode layer (bf16 natural-layout
    factors, up to 128 tokens, ranks multiples of 128) and the large-tile
    path (more than 64 tokens) run each branch at its own rank; the other
    shapes (fp8 or Linear-layout factors at decode token counts, ranks the
    decode layer's tiles do not divide) zero-pad the smaller of the gate and
    up branches, which does not change the result but costs a padded copy of
    both branches' factors (kept for the 8 most recent layers, so repeated
    calls reuse it).
    ``workspace``/``out`` may be supplied to avoid per-call allocation (see
    :func:`svd_mlp_workspace`, with r the largest rank).  ``contracted``
    asks for the contracted layer (SVDMLP_CONTRACT: h kept inside the
    kernel, taken at 1-4 tokens; other shapes run as without it).
    ``fp8_activations`` (fp8 factors only, SVDMLP_FP8_ACT): the h . Ud stage
    quantises h to e4m3 per token row and runs on the fp8 MFMA (large-tile
    path; ~2.7% relative error at the 70B shape against ~0.5% without)."""
    lib = _lib.load()
    x, ptrs, holders, flags, w_code, scale_arr, ld_arr, out, workspace, dims, dev = _prepare_layer(
        x, u_gate, v_gate, u_up, v_up, u_down, v_down, workspace, out)
    if contracted:
        flags |= _lib.SVDMLP_CONTRACT
    if fp8_activations:
        flags |= _lib.SVDMLP_FP8_ACT
    rc = _on_device(dev, lambda: lib.svdmlp_svd_mlp_ranks(
        x.data_ptr(), *ptrs,
        ctypes.addressof(scale_arr) if scale_arr is not None else None,
        ctypes.addressof(ld_arr) if ld_arr is not None else None, out.data_ptr(),
        *dims, _ACT_CODES[x.dtype], w_code, flags,
        workspace.data_ptr(), workspace.numel(), _stream(dev)))
    del holders
    if rc == _lib.SVDMLP_EUNSUP:
        return svd_mlp(x, *_pad_branches(u_gate, v_gate, u_up, v_up), u_down, v_down, workspace=workspace, out=out,
                       contracted=contracted, fp8_activations=fp8_activations)
    _lib.check(rc)
    return out


def svd_mlp_block(x, norm_weight, u_gate, v_gate, u_up, v_up, u_down, v_down, *, eps: float = 1e-5,
                  workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """One MLP block of the model, x + svd_mlp(RMSNorm(x) * norm_weight):
    LlamaRMSNorm in fp32 (models/modeling_llama.py:253-262) and the residual
    add of bench/e2e_block.py:268-278, both rounded to x.dtype.
    ``norm_weight`` is the (d,) gain (any float dtype; used in fp32)."""
    lib = _lib.load()
    x, ptrs, holders, flags, w_code, scale_arr, ld_arr, out, workspace, dims, dev = _prepare_layer(
        x, u_gate, v_gate, u_up, v_up, u_down, v_down, workspace, out)
    if out.data_ptr() == x.data_ptr():
        raise ValueError("out must not alias x")
    d = dims[1]
    if norm_weight.dim() != 1 or norm_weight.shape[0] != d or norm_weight.device != dev:
        raise ValueError(f"norm_weight must be a ({d},) tensor on x.device")
    gain = norm_weight.to(torch.float32).contiguous()
    eps = float(eps)
    if not eps > 0:
        raise ValueError(f"eps must be positive, got {eps}")
    rc = _on_device(dev, lambda: lib.svdmlp_svd_mlp_block_ranks(
        x.data_ptr(), gain.data_ptr(), eps, *ptrs,
        ctypes.addressof(scale_arr) if scale_arr is not None else None,
        ctypes.addressof(ld_arr) if ld_arr is not None else None, out.data_ptr(),
        *dims, _ACT_CODES[x.dtype], w_code, flags,
        workspace.data_ptr(), workspace.numel(), _stream(dev)))
    del holders, gain
    if rc == _lib.SVDMLP_EUNSUP:
        return svd_mlp_block(x, norm_weight, *_pad_branches(u_gate, v_gate, u_up, v_up), u_down, v_down, eps=eps,
                             workspace=workspace, out=out)
    _lib.check(rc)
    return out


def svd_mlp_workspace(x: torch.Tensor, *, r: int, ff: int, w_code: int | None = None) -> torch.Tensor:
    """Allocate the workspace svd_mlp needs for x's shape (reusable)."""
    T, d = _shape(x)
    code = _lib.SVDMLP_BF16 if w_code is None else w_code
    return _workspace(x.device, T, d, ff, r, code)


def workspace_status(workspace: torch.Tensor | None = None, *, reset: bool = False) -> bool:
    """True if a grid-barrier wait of the persistent decode kernels gave up
    in an earlier call on ``workspace`` (those calls wrote NaN into y
    wherever their result could be incomplete; the flag stays set until
    reset).  Waits for the current stream.  ``reset`` then zeroes the
    workspace's sync area, which makes it usable again.  Without a workspace,
    checks (and resets) every workspace kept for calls that pass none."""
    if workspace is None:
        return any([workspace_status(ws, reset=reset) for ws in list(_WS_CACHE.values())])
    if workspace.dtype != torch.uint8 or not workspace.is_cuda:
        raise TypeError("workspace must be a uint8 CUDA tensor from svd_mlp_workspace")
    lib = _lib.load()
    rc = lib.svdmlp_workspace_status(workspace.data_ptr(), workspace.numel(), int(bool(reset)),
                                     _stream(workspace.device))
    if rc < 0:
        _lib.check(rc)
    return rc == 1


# ---------------------------------------------------------------------------
# Host helpers of kernels/reference.py
# ---------------------------------------------------------------------------

def low_rank_dim(hidden_size: int, intermediate_size: int, compress_ratio: float) -> int:
    """SVD rank aligned to 128 (kernels/reference.py:21-34): Python's
    round-half-to-even of I*H*c / ((I+H)*128), times 128."""
    numer = intermediate_size * hidden_size * compress_ratio
    denom = (intermediate_size + hidden_size) * 128
    return round(numer / denom) * 128


def silu(x: torch.Tensor) -> torch.Tensor:
    """x * sigmoid(x) computed in float32 (kernels/reference.py:37-51)."""
    return torch.nn.functional.silu(x.float())
