"""Python entry to the gfx950 kernels through the C-ABI (include/mk_kernels.h).

torch provides device memory and the current HIP stream; every call goes
through ctypes into libmk_kernels.so.  There is no CPU or torch fallback:
if the library is missing the call raises.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

MK = dict(PRED=1, S8=2, S16=3, S32=4, S64=5, U8=6, U16=7, U32=8, U64=9,
          F16=10, F32=11, F64=12, BF16=13)

_TORCH_TO_MK = {
    torch.bool: MK["PRED"], torch.int8: MK["S8"], torch.int16: MK["S16"],
    torch.int32: MK["S32"], torch.int64: MK["S64"], torch.uint8: MK["U8"],
    torch.float16: MK["F16"], torch.float32: MK["F32"], torch.float64: MK["F64"],
    torch.bfloat16: MK["BF16"],
}
_MK_TO_TORCH = {v: k for k, v in _TORCH_TO_MK.items()}

REDUCE_OP = {"sum": 0, "max": 1, "min": 2, "prod": 3}


def mk_dtype(t: torch.dtype) -> int:
    try:
        return _TORCH_TO_MK[t]
    except KeyError as e:
        raise TypeError(f"no mk dtype for {t}") from e


def lib():
    return _lib.load_kernels()


def _stream(stream=None) -> ctypes.c_void_p:
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _check(rc, what):
    _lib.check(rc, what)


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("mk kernels take device tensors")


# ------------------------------------------------------------------ a5 attention
def sdpa_fwd(q, k, v, scale: float, causal: bool = True, out=None, lse=None, stream=None):
    """O = softmax(scale Q Kᵀ [causal tril mask]) V on [B, H, S, D] bf16 views
    (any B/H/S strides, D contiguous)."""
    _require_cuda(q, k, v)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    for t in (q, k, v):
        if t.dtype != torch.bfloat16 or t.stride(3) != 1:
            raise ValueError("sdpa_fwd: bf16 tensors with contiguous head_dim")
    if out is None:
        out = torch.empty((B, H, Sq, D), dtype=torch.bfloat16, device=q.device)
    rc = lib().mk_sdpa_fwd(
        _stream(stream), B, H, Sq, Sk, D,
        _ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        _ptr(out), out.stride(0), out.stride(1), out.stride(2),
        float(scale), int(bool(causal)), _ptr(lse))
    _check(rc, "mk_sdpa_fwd")
    return out


# ------------------------------------------------------------------ a4 GEMM
def gemm(a, b, out_dtype=None, bias=None, relu=False, out=None, stream=None):
    """C[b] = A[b] @ B[b] (+bias)(relu) for 2-D or 3-D views with a unit
    stride along one dim of each operand (transposed views are free)."""
    _require_cuda(a, b)
    if a.dtype != b.dtype:
        raise ValueError("gemm: operand dtypes differ")
    squeeze = a.dim() == 2
    a3 = a.unsqueeze(0) if squeeze else a
    b3 = b.unsqueeze(0) if b.dim() == 2 else b
    batch, M, K = a3.shape
    _, K2, N = b3.shape
    if K2 != K:
        raise ValueError("gemm: inner dims differ")
    out_dtype = out_dtype or a.dtype
    if out is None:
        out = torch.empty((batch, M, N), dtype=out_dtype, device=a.device)
    o3 = out.unsqueeze(0) if out.dim() == 2 else out
    b_bs = b3.stride(0) if b3.shape[0] == batch and b.dim() == 3 else 0
    epi = 0 if bias is None else (2 if relu else 1)
    if bias is not None and bias.dtype == torch.float32 and out_dtype != torch.float32:
        epi |= 4  # an fp32 bias added before the narrowing store
    rc = lib().mk_gemm(
        _stream(stream), mk_dtype(a.dtype), mk_dtype(out_dtype), batch, M, N, K,
        _ptr(a3), a3.stride(0), a3.stride(1), a3.stride(2),
        _ptr(b3), b_bs, b3.stride(1), b3.stride(2),
        _ptr(o3), o3.stride(0), o3.stride(1), _ptr(bias), epi)
    _check(rc, "mk_gemm")
    return out[0] if squeeze and out.dim() == 3 else out


# ------------------------------------------------------------------ a8/a9 reductions
def row_reduce(x, op="sum", out_dtype=torch.float32, init=None, stream=None):
    _require_cuda(x)
    x = x.contiguous()
    rows = x.numel() // x.shape[-1] if x.numel() else 0
    y = torch.empty(x.shape[:-1], dtype=out_dtype, device=x.device)
    if init is None:
        init = {"sum": 0.0, "max": float("-inf"), "min": float("inf"), "prod": 1.0}[op]
    rc = lib().mk_row_reduce(_stream(stream), mk_dtype(x.dtype), mk_dtype(out_dtype),
                             REDUCE_OP[op], rows, x.shape[-1], _ptr(x), float(init), _ptr(y))
    _check(rc, "mk_row_reduce")
    return y


def row_argmax(x, is_min=False, index_dtype=torch.int32, with_values=True, stream=None):
    _require_cuda(x)
    x = x.contiguous()
    rows = x.numel() // x.shape[-1] if x.numel() else 0
    idx = torch.empty(x.shape[:-1], dtype=index_dtype, device=x.device)
    vals = torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device) if with_values else None
    rc = lib().mk_row_argmax(_stream(stream), mk_dtype(x.dtype), int(is_min), rows, x.shape[-1],
                             _ptr(x), _ptr(vals), mk_dtype(index_dtype), _ptr(idx))
    _check(rc, "mk_row_argmax")
    return idx, vals


def layernorm(x, gamma=None, beta=None, eps=1e-5, out_dtype=None, stream=None):
    """LayerNorm over the last axis; out_dtype (default x's) may be bf16 for
    fp32 x (mk_layernorm_typed)."""
    _require_cuda(x)
    x = x.contiguous()
    out_dtype = x.dtype if out_dtype is None else out_dtype
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    rows = x.numel() // x.shape[-1]
    rc = lib().mk_layernorm_typed(_stream(stream), mk_dtype(x.dtype), mk_dtype(out_dtype), rows, x.shape[-1],
                                  _ptr(x), _ptr(gamma), _ptr(beta), float(eps), _ptr(y))
    _check(rc, "mk_layernorm_typed")
    return y


def softmax_rows(x, stream=None):
    _require_cuda(x)
    x = x.contiguous()
    y = torch.empty_like(x)
    rows = x.numel() // x.shape[-1]
    rc = lib().mk_softmax_rows(_stream(stream), mk_dtype(x.dtype), rows, x.shape[-1], _ptr(x), _ptr(y))
    _check(rc, "mk_softmax_rows")
    return y


# ------------------------------------------------------------------ a7 elementwise
def gelu_tanh(x, out=None, stream=None):
    _require_cuda(x)
    x = x.contiguous()
    y = torch.empty_like(x) if out is None else out
    rc = lib().mk_gelu_tanh(_stream(stream), mk_dtype(x.dtype), x.numel(), _ptr(x), _ptr(y))
    _check(rc, "mk_gelu_tanh")
    return y


def convert(x, dtype, stream=None):
    _require_cuda(x)
    x = x.contiguous()
    y = torch.empty(x.shape, dtype=dtype, device=x.device)
    rc = lib().mk_convert(_stream(stream), mk_dtype(x.dtype), mk_dtype(dtype), x.numel(), _ptr(x), _ptr(y))
    _check(rc, "mk_convert")
    return y


def fill(out, pattern: int, stream=None):
    rc = lib().mk_fill(_stream(stream), out.element_size(), out.numel(), ctypes.c_uint64(pattern), _ptr(out))
    _check(rc, "mk_fill")
    return out


def iota(shape, dim, dtype=torch.int32, device="cuda", stream=None):
    out = torch.empty(shape, dtype=dtype, device=device)
    dims = (ctypes.c_int64 * len(shape))(*shape)
    rc = lib().mk_iota(_stream(stream), mk_dtype(dtype), len(shape), dims, dim, _ptr(out))
    _check(rc, "mk_iota")
    return out


def copy_strided(x, stream=None):
    """Materialise any strided view (transpose / broadcast via expand) densely."""
    _require_cuda(x)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    r = x.dim()
    dims = (ctypes.c_int64 * max(r, 1))(*x.shape)
    strides = (ctypes.c_int64 * max(r, 1))(*x.stride())
    rc = lib().mk_copy_strided(_stream(stream), x.element_size(), r, dims, _ptr(x), strides, _ptr(out))
    _check(rc, "mk_copy_strided")
    return out


_EW_NAMES = ("CONST ADD SUB MUL DIV MAX MIN POW NEG EXP LOG TANH SQRT RSQRT ABS LOGISTIC "
             "CMP_EQ CMP_NE CMP_LT CMP_LE CMP_GT CMP_GE SELECT CLAMP ROUND_BF16 ROUND_F16 FLOOR "
             "CEIL SIGN AND OR NOT MOV CMP_LT_S32 CMP_GE_S32 ADD_S32 SUB_S32 MUL_S32 S32_TO_F32 "
             "F32_TO_S32 ERF CMP_EQ_S32 CMP_NE_S32 CMP_LE_S32 CMP_GT_S32 MAX_S32 MIN_S32 NEG_S32 "
             "AND_B32 OR_B32 XOR_B32 PRED_TO_S32 S32_TO_PRED U32_TO_F32").split()
EW = {n: i for i, n in enumerate(_EW_NAMES)}  # mirrors enum mk_ew_op in include/mk_kernels.h


def ew_program(shape, inputs, program, consts, out_reg, out_dtype, stream=None, out=None):
    """Run a fused elementwise program.  `inputs` are tensors broadcast (via
    torch.expand views) to `shape`; `program` is a list of (op, dst, a, b);
    `out` (optional) a dense tensor of `shape` and `out_dtype` to write."""
    rank = len(shape)
    dev = inputs[0].device if inputs else "cuda"
    if out is None:
        out = torch.empty(shape, dtype=out_dtype, device=dev)
    elif tuple(out.shape) != tuple(shape) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("ew_program: out must be a dense tensor of the given shape and dtype")
    ptrs = (ctypes.c_void_p * max(len(inputs), 1))(*[t.data_ptr() for t in inputs])
    types = (ctypes.c_int * max(len(inputs), 1))(*[mk_dtype(t.dtype) for t in inputs])
    strides = (ctypes.c_int64 * (6 * max(len(inputs), 1)))()
    for i, t in enumerate(inputs):
        tt = t.expand(shape)
        for d in range(rank):
            strides[6 * i + d] = tt.stride(d)
    prog = (ctypes.c_int32 * (4 * max(len(program), 1)))()
    for p, ins in enumerate(program):
        for j in range(4):
            prog[4 * p + j] = int(ins[j])
    cst = (ctypes.c_float * max(len(consts), 1))(*consts)
    dims = (ctypes.c_int64 * max(rank, 1))(*shape)
    rc = lib().mk_ew_program(_stream(stream), rank, dims, len(inputs), ptrs, types, strides,
                             len(program), prog, cst, len(consts), out_reg, mk_dtype(out_dtype),
                             _ptr(out))
    _check(rc, "mk_ew_program")
    return out


def ew_program_multi(shape, inputs, program, consts, out_regs, outs, stream=None):
    """mk_ew_program_multi: one program, 1 to 4 outputs (dense tensors of
    `shape`, each written from its register in out_regs)."""
    rank = len(shape)
    for o in outs:
        if tuple(o.shape) != tuple(shape) or not o.is_contiguous():
            raise ValueError("ew_program_multi: outputs must be dense tensors of the given shape")
    ptrs = (ctypes.c_void_p * max(len(inputs), 1))(*[t.data_ptr() for t in inputs])
    types = (ctypes.c_int * max(len(inputs), 1))(*[mk_dtype(t.dtype) for t in inputs])
    strides = (ctypes.c_int64 * (6 * max(len(inputs), 1)))()
    for i, t in enumerate(inputs):
        tt = t.expand(shape)
        for d in range(rank):
            strides[6 * i + d] = tt.stride(d)
    prog = (ctypes.c_int32 * (4 * max(len(program), 1)))()
    for p, ins in enumerate(program):
        for j in range(4):
            prog[4 * p + j] = int(ins[j])
    cst = (ctypes.c_float * max(len(consts), 1))(*consts)
    dims = (ctypes.c_int64 * max(rank, 1))(*shape)
    regs = (ctypes.c_int * len(outs))(*out_regs)
    otypes = (ctypes.c_int * len(outs))(*[mk_dtype(o.dtype) for o in outs])
    optrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    rc = lib().mk_ew_program_multi(_stream(stream), rank, dims, len(inputs), ptrs, types, strides, len(program),
                                   prog, cst, len(consts), len(outs), regs, otypes, optrs)
    _check(rc, "mk_ew_program_multi")
    return outs


# ------------------------------------------------------------------ a10/a11 indexing
def gather_rows(table, ids, stream=None):
    _require_cuda(table, ids)
    table = table.contiguous()
    ids_c = ids.contiguous()
    out = torch.empty(tuple(ids.shape) + tuple(table.shape[1:]), dtype=table.dtype, device=table.device)
    row_bytes = table[0].numel() * table.element_size() if table.shape[0] else 0
    rc = lib().mk_gather_rows(_stream(stream), table.shape[0], row_bytes, _ptr(table),
                              mk_dtype(ids.dtype), ids_c.numel(), _ptr(ids_c), _ptr(out))
    _check(rc, "mk_gather_rows")
    return out


def scatter_add_rows(table, ids, updates, out=None, workspace=None, stream=None):
    """out[r] = table[r] + sum_{i: ids[i]==r, in increasing i} updates[i]
    (bit-exact sequential order); out may be `table` itself (in place)."""
    _require_cuda(table, ids, updates)
    ids_c = ids.contiguous().reshape(-1)
    n_rows, row_len = table.shape[0], table[0].numel()
    if out is None:
        out = torch.empty_like(table)
    nbytes = lib().mk_scatter_add_workspace_bytes(n_rows, ids_c.numel())
    if workspace is None:
        workspace = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=table.device)
    elif workspace.numel() < nbytes:
        raise ValueError("scatter_add_rows: workspace too small")
    rc = lib().mk_scatter_add_rows(_stream(stream), mk_dtype(table.dtype), n_rows, row_len,
                                   _ptr(table), mk_dtype(ids.dtype), ids_c.numel(), _ptr(ids_c),
                                   _ptr(updates.contiguous()), _ptr(out), _ptr(workspace))
    _check(rc, "mk_scatter_add_rows")
    return out


def scatter_add_rows_noalloc(table, ids, updates, out=None, stream=None):
    """scatter_add_rows through mk_scatter_add_rows_noalloc: no workspace and
    no device allocation inside the call (the library's fixed per-GPU
    scratch array, MK_SCATTER_ADD_SCRATCH_BYTES, is used instead)."""
    _require_cuda(table, ids, updates)
    ids_c = ids.contiguous().reshape(-1)
    n_rows, row_len = table.shape[0], table[0].numel()
    if out is None:
        out = torch.empty_like(table)
    rc = lib().mk_scatter_add_rows_noalloc(_stream(stream), mk_dtype(table.dtype), n_rows, row_len,
                                           _ptr(table), mk_dtype(ids.dtype), ids_c.numel(), _ptr(ids_c),
                                           _ptr(updates.contiguous()), _ptr(out))
    _check(rc, "mk_scatter_add_rows_noalloc")
    return out


# ------------------------------------------------------------------ C5 training step
def _ws(nbytes, device, workspace):
    if workspace is None:
        return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
    if workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError("workspace too small")
    return workspace


def _mat_strides(t):
    """(batch stride, row stride, column stride) of a 2-D or 3-D view."""
    if t.dim() == 2:
        return 0, t.stride(0), t.stride(1)
    return t.stride(0), t.stride(1), t.stride(2)


def gemm_blas(a, b, out=None, out_dtype=None, alpha=1.0, beta=0.0, stream=None):
    """out = alpha a @ b + beta out through rocBLAS (mk_gemm_blas); a [.., M, K],
    b [.., K, N] views with one unit stride each (either orientation)."""
    _require_cuda(a, b)
    M, Kd = a.shape[-2:]
    N = b.shape[-1]
    batch = a.shape[0] if a.dim() == 3 else 1
    if out is None:
        shape = (batch, M, N) if a.dim() == 3 else (M, N)
        out = torch.zeros(shape, dtype=out_dtype or a.dtype, device=a.device)
    a_bs, a_ms, a_ks = _mat_strides(a)
    b_bs, b_ks, b_ns = _mat_strides(b)
    c_bs, c_ms, _ = _mat_strides(out)
    rc = lib().mk_gemm_blas(_stream(stream), mk_dtype(a.dtype), mk_dtype(out.dtype), batch, M, N, Kd, _ptr(a), a_bs,
                            a_ms, a_ks, _ptr(b), b_bs, b_ks, b_ns, _ptr(out), c_bs, c_ms, float(alpha), float(beta))
    _check(rc, "mk_gemm_blas")
    return out


def gemm_bias_gelu(a, b, bias=None, out_dtype=torch.bfloat16, out=None, y=None, stream=None):
    """(C, Y): C = a @ b (+ bias) in out_dtype and Y = bf16 gelu_tanh(C as
    stored), one launch (mk_gemm_bias_gelu); a [M, K], b [K, N] 2-D views."""
    _require_cuda(a, b)
    M, Kd = a.shape
    N = b.shape[1]
    out = torch.empty(M, N, dtype=out_dtype, device=a.device) if out is None else out
    y = torch.empty(M, N, dtype=torch.bfloat16, device=a.device) if y is None else y
    epi = 0 if bias is None else (5 if bias.dtype == torch.float32 and out.dtype != torch.float32 else 1)
    rc = lib().mk_gemm_bias_gelu(_stream(stream), mk_dtype(a.dtype), mk_dtype(out.dtype), M, N, Kd, _ptr(a),
                                 a.stride(0), a.stride(1), _ptr(b), b.stride(0), b.stride(1), _ptr(out),
                                 out.stride(0), _ptr(bias), epi, _ptr(y), y.stride(0))
    _check(rc, "mk_gemm_bias_gelu")
    return out, y


def gemm_gelu_bwd(a, b, pre, out=None, workspace=None, stream=None):
    """(dx, dx column sums): dx = bf16(bf16(a @ b) * gelu_tanh'(pre)) and its
    fp32 column sums, one GEMM launch plus a column pass
    (mk_gemm_gelu_bwd); a [M, K], b [K, N], pre [M, N] bf16 2-D views."""
    _require_cuda(a, b, pre)
    M, Kd = a.shape
    N = b.shape[1]
    out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device) if out is None else out
    colsum = torch.empty(N, dtype=torch.float32, device=a.device)
    ws = _ws(lib().mk_gemm_gelu_bwd_workspace_bytes(M, N), a.device, workspace)
    rc = lib().mk_gemm_gelu_bwd(_stream(stream), mk_dtype(a.dtype), M, N, Kd, _ptr(a), a.stride(0), a.stride(1),
                                _ptr(b), b.stride(0), b.stride(1), _ptr(out), out.stride(0), _ptr(pre), pre.stride(0),
                                _ptr(colsum), _ptr(ws))
    _check(rc, "mk_gemm_gelu_bwd")
    return out, colsum


def gemm_splitk(a, b, splits, out=None, workspace=None, stream=None, out_dtype=torch.float32, bias=None,
                relu=False):
    """out = a @ b (+ bias)(ReLU) with the contraction cut into `splits`
    slices summed in order in fp32 (mk_gemm_splitk; mk_gemm_splitk_typed for
    a bf16 `out_dtype`, a bias or a K that `splits` does not divide);
    a [M, K], b [K, N] 2-D views."""
    _require_cuda(a, b)
    M, Kd = a.shape
    N = b.shape[1]
    out = torch.empty(M, N, dtype=out_dtype, device=a.device) if out is None else out
    ws = _ws(lib().mk_gemm_splitk_workspace_bytes(M, N, splits), a.device, workspace)
    if out.dtype == torch.float32 and Kd % splits == 0 and bias is None:
        rc = lib().mk_gemm_splitk(_stream(stream), mk_dtype(a.dtype), M, N, Kd, _ptr(a), a.stride(0), a.stride(1),
                                  _ptr(b), b.stride(0), b.stride(1), _ptr(out), out.stride(0), splits, _ptr(ws))
        _check(rc, "mk_gemm_splitk")
        return out
    rc = lib().mk_gemm_splitk_typed(_stream(stream), mk_dtype(a.dtype), mk_dtype(out.dtype), M, N, Kd, _ptr(a),
                                    a.stride(0), a.stride(1), _ptr(b), b.stride(0), b.stride(1), _ptr(out),
                                    out.stride(0), splits, _ptr(ws), _ptr(bias),
                                    0 if bias is None else ((2 if relu else 1) |
                                                            (4 if bias.dtype != out.dtype else 0)))
    _check(rc, "mk_gemm_splitk_typed")
    return out


def gemm_blas_splitk(a, b, splits, out=None, workspace=None, stream=None):
    """fp32 out = a @ b with the contraction cut into `splits` slices
    (mk_gemm_blas_splitk); a [M, K], b [K, N] 2-D views."""
    _require_cuda(a, b)
    M, Kd = a.shape
    N = b.shape[1]
    out = torch.empty(M, N, dtype=torch.float32, device=a.device) if out is None else out
    ws = _ws(lib().mk_gemm_blas_splitk_workspace_bytes(M, N, splits), a.device, workspace)
    rc = lib().mk_gemm_blas_splitk(_stream(stream), mk_dtype(a.dtype), M, N, Kd, _ptr(a), a.stride(0), a.stride(1),
                                   _ptr(b), b.stride(0), b.stride(1), _ptr(out), out.stride(0), splits, _ptr(ws))
    _check(rc, "mk_gemm_blas_splitk")
    return out


def add_rows(a, b=None, bias=None, out=None, stream=None):
    """out = a + b + bias (bias broadcast over the rows of a 2-D a), one pass
    with fp32 math and one rounding; b and bias are optional, out may be a or b."""
    _require_cuda(a)
    rows, cols = a.shape
    for t in (b, bias):
        if t is not None:
            _require_cuda(t)
            if t.dtype != a.dtype or not t.is_contiguous():
                raise ValueError("add_rows: operands must share a's dtype and be contiguous")
    if b is not None and b.shape != a.shape:
        raise ValueError("add_rows: b must have a's shape")
    if bias is not None and bias.numel() != cols:
        raise ValueError("add_rows: bias must have one value per column")
    out = torch.empty_like(a) if out is None else out
    rc = lib().mk_add_rows(_stream(stream), mk_dtype(a.dtype), rows, cols, _ptr(a), _ptr(b), _ptr(bias), _ptr(out))
    _check(rc, "mk_add_rows")
    return out


def add_layernorm(a, b, bias, gamma, beta, eps=1e-5, sum_out=None, y=None, out_dtype=None, stream=None):
    """(a + b + bias, LayerNorm of that sum) for [rows, cols] a, b: bf16 rows
    (mk_add_layernorm), or fp32 rows without a bias and an fp32 or bf16
    LayerNorm (mk_add_layernorm_typed)."""
    _require_cuda(a)
    rows, cols = a.shape
    out_dtype = a.dtype if out_dtype is None else out_dtype
    sum_out = torch.empty_like(a) if sum_out is None else sum_out
    y = torch.empty(a.shape, dtype=out_dtype, device=a.device) if y is None else y
    rc = lib().mk_add_layernorm_typed(_stream(stream), mk_dtype(a.dtype), mk_dtype(y.dtype), rows, cols, _ptr(a),
                                      _ptr(b), _ptr(bias), _ptr(gamma), _ptr(beta), float(eps), _ptr(sum_out), _ptr(y))
    _check(rc, "mk_add_layernorm_typed")
    return sum_out, y


def bias_gelu(x, bias, pre_out=None, y=None, stream=None):
    """(x + bias, gelu_tanh of that sum) for bf16 [rows, cols] x."""
    _require_cuda(x, bias)
    rows, cols = x.shape
    pre_out = torch.empty_like(x) if pre_out is None else pre_out
    y = torch.empty_like(x) if y is None else y
    rc = lib().mk_bias_gelu(_stream(stream), rows, cols, _ptr(x), _ptr(bias), _ptr(pre_out), _ptr(y))
    _check(rc, "mk_bias_gelu")
    return pre_out, y


def gelu_tanh_bwd(x, dy, out=None, stream=None):
    """dx = dy * gelu_tanh'(x) (same dtype as x; out may be dy)."""
    _require_cuda(x, dy)
    out = torch.empty_like(x) if out is None else out
    rc = lib().mk_gelu_tanh_bwd(_stream(stream), mk_dtype(x.dtype), x.numel(), _ptr(x), _ptr(dy), _ptr(out))
    _check(rc, "mk_gelu_tanh_bwd")
    return out


def col_sum(x, out=None, workspace=None, stream=None):
    """fp32 column sums of a 2-D (rows, cols) contiguous tensor."""
    _require_cuda(x)
    rows, cols = x.shape
    out = torch.empty(cols, dtype=torch.float32, device=x.device) if out is None else out
    ws = _ws(lib().mk_col_sum_workspace_bytes(rows, cols), x.device, workspace)
    rc = lib().mk_col_sum(_stream(stream), mk_dtype(x.dtype), rows, cols, _ptr(x), _ptr(out), _ptr(ws))
    _check(rc, "mk_col_sum")
    return out


def layernorm_bwd(x, gamma, dy, eps=1e-5, dx=None, dgamma=None, dbeta=None, workspace=None, want_params=True,
                  dres=None, want_colsum=False, dx_bf16=None, stream=None):
    """(dx, dgamma, dbeta[, dx_colsum]) of LayerNorm over the last axis (fp32
    dgamma/dbeta/colsum); dx = LN'(dy) + dres when dres is given; dx_bf16
    (fp32 rows) also receives dx rounded to bf16."""
    _require_cuda(x, dy)
    cols = x.shape[-1]
    rows = x.numel() // cols
    dx = torch.empty_like(x) if dx is None else dx
    if want_params:
        dgamma = torch.empty(cols, dtype=torch.float32, device=x.device) if dgamma is None else dgamma
        dbeta = torch.empty(cols, dtype=torch.float32, device=x.device) if dbeta is None else dbeta
    colsum = torch.empty(cols, dtype=torch.float32, device=x.device) if want_colsum else None
    ws = _ws(lib().mk_layernorm_bwd_workspace_bytes(rows, cols), x.device, workspace)
    rc = lib().mk_layernorm_bwd_typed(_stream(stream), mk_dtype(x.dtype), rows, cols, _ptr(x), _ptr(gamma),
                                      _ptr(dy), _ptr(dres), float(eps), _ptr(dx), _ptr(dx_bf16),
                                      _ptr(dgamma if want_params else None), _ptr(dbeta if want_params else None),
                                      _ptr(colsum), _ptr(ws))
    _check(rc, "mk_layernorm_bwd_typed")
    return (dx, dgamma, dbeta, colsum) if want_colsum else (dx, dgamma, dbeta)


def gelu_tanh_bwd_colsum(x, dy, out=None, workspace=None, stream=None):
    """(dx, dx column sums in fp32) of dx = dy * gelu_tanh'(x) on 2-D x."""
    _require_cuda(x, dy)
    rows, cols = x.shape
    out = torch.empty_like(x) if out is None else out
    colsum = torch.empty(cols, dtype=torch.float32, device=x.device)
    ws = _ws(lib().mk_col_sum_workspace_bytes(rows, cols), x.device, workspace)
    rc = lib().mk_gelu_tanh_bwd_colsum(_stream(stream), mk_dtype(x.dtype), rows, cols, _ptr(x), _ptr(dy), _ptr(out),
                                       _ptr(colsum), _ptr(ws))
    _check(rc, "mk_gelu_tanh_bwd_colsum")
    return out, colsum


def softmax_xent(logits, labels, grad_scale, loss_rows=None, dlogits=None, stream=None):
    """Per-row softmax cross-entropy loss (fp32) and the logit gradient
    (dlogits may be logits itself; a bf16 dlogits for fp32 logits takes the
    mixed-type kernel)."""
    _require_cuda(logits, labels)
    cols = logits.shape[-1]
    rows = logits.numel() // cols
    loss_rows = torch.empty(rows, dtype=torch.float32, device=logits.device) if loss_rows is None else loss_rows
    dlogits = torch.empty_like(logits) if dlogits is None else dlogits
    if logits.dim() == 2 and (logits.stride(0) != cols or dlogits.stride(0) != cols):
        # row pitches of 2-D views (padded rows): mk_softmax_xent_strided
        if logits.stride(1) != 1 or dlogits.stride(1) != 1 or dlogits.shape != logits.shape:
            raise ValueError("softmax_xent: rows must be contiguous")
        rc = lib().mk_softmax_xent_strided(_stream(stream), mk_dtype(logits.dtype), mk_dtype(dlogits.dtype), rows,
                                           cols, _ptr(logits), logits.stride(0), mk_dtype(labels.dtype),
                                           _ptr(labels), float(grad_scale), _ptr(loss_rows), _ptr(dlogits),
                                           dlogits.stride(0))
        _check(rc, "mk_softmax_xent_strided")
        return loss_rows, dlogits
    rc = lib().mk_softmax_xent_typed(_stream(stream), mk_dtype(logits.dtype), mk_dtype(dlogits.dtype), rows, cols,
                                     _ptr(logits), mk_dtype(labels.dtype), _ptr(labels), float(grad_scale),
                                     _ptr(loss_rows), _ptr(dlogits))
    _check(rc, "mk_softmax_xent_typed")
    return loss_rows, dlogits


def adam_update(param, grad, m, v, lr, b1, b2, eps, bc1, bc2, master=None, stream=None):
    """One Adam step in place (temp/dp_train.py:71-75 semantics)."""
    rc = lib().mk_adam_update(_stream(stream), param.numel(), mk_dtype(param.dtype), _ptr(param), _ptr(master),
                              mk_dtype(grad.dtype), _ptr(grad), _ptr(m), _ptr(v), float(lr), float(b1),
                              float(b2), float(eps), float(bc1), float(bc2))
    _check(rc, "mk_adam_update")


def adam_update_dev(param, grad, m, v, hyper, b1, b2, eps, master=None, stream=None):
    """adam_update with hyper = device fp32 tensor [lr, bc1, bc2]."""
    rc = lib().mk_adam_update_dev(_stream(stream), param.numel(), mk_dtype(param.dtype), _ptr(param), _ptr(master),
                                  mk_dtype(grad.dtype), _ptr(grad), _ptr(m), _ptr(v), _ptr(hyper), float(b1),
                                  float(b2), float(eps))
    _check(rc, "mk_adam_update_dev")


def sdpa_bwd(q, k, v, o, dout, lse, scale, causal=True, dq=None, dk=None, dv=None, workspace=None, stream=None):
    """(dq, dk, dv) of mk_sdpa_fwd on [B, H, S, D] bf16 views."""
    _require_cuda(q, k, v, o, dout, lse)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(v) if dv is None else dv
    ws = _ws(lib().mk_sdpa_bwd_workspace_bytes(B, H, Sq, Sk, D), q.device, workspace)
    args = [_stream(stream), B, H, Sq, Sk, D]
    for t in (q, k, v, o, dout):
        args += [_ptr(t), t.stride(0), t.stride(1), t.stride(2)]
    args += [_ptr(lse)]
    for t in (dq, dk, dv):
        args += [_ptr(t), t.stride(0), t.stride(1), t.stride(2)]
    args += [float(scale), int(bool(causal)), _ptr(ws)]
    rc = lib().mk_sdpa_bwd(*args)
    _check(rc, "mk_sdpa_bwd")
    return dq, dk, dv
