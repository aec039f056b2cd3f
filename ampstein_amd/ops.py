"""The reference's EXL3 operator interface over torch tensors, backed by libexl3_amd.so.

Names, argument order, argument meaning and error behaviour follow the vendored
exllamav3 functions that ampstein's torch.so binds (argument checks raise, as TORCH_CHECK
does; nothing falls back to a CPU path):

  reconstruct            vendor/exl3/exllamav3_ext/quant/reconstruct.cu:492-501
  reconstruct_slice      vendor/exl3/exllamav3_ext/quant/reconstruct.cu:141-194
  reconstruct_had_slice  vendor/exl3/exllamav3_ext/quant/reconstruct.cu:431-490
  had_r_128              vendor/exl3/exllamav3_ext/quant/hadamard.cu:125-210
  exl3_gemm              vendor/exl3/exllamav3_ext/quant/exl3_gemm.cu:114-350
  exl3_gemm_recon        src/torch/amp_torch.cpp:11149-11230 (prefill policy)

Tensors stay on the caller's device; work is enqueued on torch's current stream.
"""
from __future__ import annotations

from typing import Optional

import os

import torch

from . import _lib
from ._lib import check

Tensor = torch.Tensor

# Row count from which exl3_gemm_recon reconstructs the weight in the original basis (one fused
# W, y = x @ W) instead of rotating x and y around W_hat: 2048, the reference's switch
# (amp_torch.cpp:11203-11209, models.uc:36-37), so the two branches round where the reference's
# do.  On MI355X the rotated form is faster at every measured size (reconstruct_had is ALU-bound,
# the activation rotations are HBM-bound and short): AMP_RECON_FUSED_ROWS=0 never takes the fused
# branch (the opt-in MI355X routing).
RECON_FUSED_ROWS = int(os.environ.get("AMP_RECON_FUSED_ROWS", "2048")) or (1 << 30)
# The fused branch's x (the caller's, row-major) is copied into k slabs before the GEMM from this
# many weight columns on: the copy costs ~ rows x k, the faster GEMM saves ~ rows x k x n (at
# 2048 rows, measured: +4 % with the copy at 8192 -> 28672, -4 % at 28672 -> 8192).
RECON_FUSED_X_SLABS_MIN_N = 16384

def _ptr(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(cond: bool, msg: str):
    if not cond:
        raise _lib.Exl3Error(_lib.EINVAL, msg)


def _dtype(t: Tensor, dt, name: str):
    _need(t.dtype == dt, f"{name} is incorrect datatype, must be {dt}")


def _cuda(*ts):
    for t in ts:
        if t is not None:
            _need(t.is_cuda, "tensors must be on a GPU device")
            _need(t.is_contiguous(), "tensors must be contiguous")


def _trellis_dtype(t: Tensor, name: str):
    _need(t.dtype in (torch.int16, torch.uint16), f"{name} is incorrect datatype, must be int16")


def _codebook_flags(mcg: bool, mul1: bool):
    _need(not (mcg and mul1), "Specified both mcg and mul1")
    return int(bool(mcg)), int(bool(mul1))


def bits_from_K(K: float):
    """quant/bits_k.cuh:178-185: integer 1..8, or 1.5 / 2.5 / 3.5."""
    bits = int(K)
    f = float(K) - bits
    _need(1 <= bits <= 8 and (f == 0.0 or (f == 0.5 and bits <= 3)),
          f"Unsupported EXL3 bitrate {K} (integer 1..8, or 1.5 / 2.5 / 3.5)")
    return bits, f == 0.5


def reconstruct_slice(unpacked: Tensor, packed: Tensor, K: float, mcg: bool, mul1: bool,
                      n_offset: int) -> None:
    """Decode trellis columns [n_offset, n_offset + unpacked.size(1)) into `unpacked`
    (fp16, rotated basis), bit-exact with the reference."""
    bits, half = bits_from_K(K)
    _need(not half or mul1, "reconstruct: half-integer bitrates require the mul1 codebook")
    _need(packed.dim() == 3 and unpacked.dim() == 2, "reconstruct: bad tensor ranks")
    _need(unpacked.size(0) == packed.size(0) * 16, "unpacked and packed shapes are incompatible")
    _need(packed.size(2) == 16 * bits + (8 if half else 0), "packed tile size does not match K")
    _dtype(unpacked, torch.half, "unpacked")
    _trellis_dtype(packed, "packed")
    if unpacked.numel() == 0:
        return
    _cuda(unpacked, packed)
    mcg_i, mul1_i = int(bool(mcg)), int(bool(mul1))     # mcg wins when both are set
    with torch.cuda.device(unpacked.device):
        check(_lib.lib().exl3_amd_reconstruct(
            unpacked.data_ptr(), packed.data_ptr(), unpacked.size(0), packed.size(1) * 16,
            unpacked.size(1), int(n_offset), float(K), mcg_i, mul1_i, _stream(unpacked)))


def reconstruct_t(unpacked_t: Tensor, packed: Tensor, K: float, mcg: bool = False,
                  mul1: bool = False, n_offset: int = 0, svh: Optional[Tensor] = None) -> None:
    """W_hat columns [n_offset, n_offset + unpacked_t.size(0)) transposed into `unpacked_t`
    (rows, k) fp16: the k-contiguous layout the recon GEMM reads fastest.  Values bit-exact
    with reconstruct (no reference counterpart: the reference keeps W (k, n) for cuBLAS,
    amp_torch.cpp:11199-11214).  With svh (the full (n) vector) the output rotation is folded in:
    (W_hat H128 diag(svh) / sqrt(128))^T, one fp16 rounding."""
    bits, half = bits_from_K(K)
    _need(not half or mul1, "reconstruct: half-integer bitrates require the mul1 codebook")
    _need(packed.dim() == 3 and unpacked_t.dim() == 2, "reconstruct: bad tensor ranks")
    _need(unpacked_t.size(1) == packed.size(0) * 16 and n_offset >= 0
          and n_offset + unpacked_t.size(0) <= packed.size(1) * 16,
          "unpacked and packed shapes are incompatible")
    _need(packed.size(2) == 16 * bits + (8 if half else 0), "packed tile size does not match K")
    _dtype(unpacked_t, torch.half, "unpacked")
    _trellis_dtype(packed, "packed")
    if unpacked_t.numel() == 0:
        return
    _cuda(unpacked_t, packed, svh)
    with torch.cuda.device(unpacked_t.device):
        if svh is not None:
            _dtype(svh, torch.half, "svh")
            _need(svh.numel() >= packed.size(1) * 16, "svh too short")
            check(_lib.lib().exl3_amd_reconstruct_t_had(
                unpacked_t.data_ptr(), packed.data_ptr(), svh.data_ptr(), unpacked_t.size(1), packed.size(1) * 16,
                unpacked_t.size(0), int(n_offset), float(K), int(bool(mcg)), int(bool(mul1)), _stream(unpacked_t)))
            return
        check(_lib.lib().exl3_amd_reconstruct_t(
            unpacked_t.data_ptr(), packed.data_ptr(), unpacked_t.size(1), packed.size(1) * 16,
            unpacked_t.size(0), int(n_offset), float(K), int(bool(mcg)), int(bool(mul1)), _stream(unpacked_t)))


def reconstruct(unpacked: Tensor, packed: Tensor, K: float, mcg: bool = False,
                mul1: bool = False) -> None:
    _need(unpacked.dim() == 2 and packed.dim() == 3 and unpacked.size(1) == packed.size(1) * 16,
          "unpacked and packed shapes are incompatible")
    reconstruct_slice(unpacked, packed, K, mcg, mul1, 0)


def reconstruct_had_slice(unpacked: Tensor, packed: Tensor, suh: Tensor, svh: Tensor,
                          K: float, mcg: bool, mul1: bool, n_offset: int) -> None:
    """Original-basis weights diag(suh) H W_hat H diag(svh) per 128x128 block."""
    bits, half = bits_from_K(K)
    _need(not half or mul1, "reconstruct: half-integer bitrates require the mul1 codebook")
    _need(packed.dim() == 3 and unpacked.dim() == 2, "reconstruct_had: bad tensor ranks")
    _need(unpacked.size(0) == packed.size(0) * 16, "unpacked and packed shapes are incompatible")
    _need(packed.size(2) == 16 * bits + (8 if half else 0), "packed tile size does not match K")
    _dtype(unpacked, torch.half, "unpacked")
    _dtype(suh, torch.half, "suh")
    _dtype(svh, torch.half, "svh")
    _trellis_dtype(packed, "packed")
    if unpacked.numel() == 0:
        return
    _need(suh.numel() >= unpacked.size(0), "reconstruct_had: suh size")
    _need(svh.numel() >= unpacked.size(1), "reconstruct_had: svh size")
    _cuda(unpacked, packed, suh, svh)
    mcg_i, mul1_i = int(bool(mcg)), int(bool(mul1))     # mcg wins when both are set
    with torch.cuda.device(unpacked.device):
        check(_lib.lib().exl3_amd_reconstruct_had(
            unpacked.data_ptr(), packed.data_ptr(), suh.data_ptr(), svh.data_ptr(),
            unpacked.size(0), packed.size(1) * 16, unpacked.size(1), int(n_offset), float(K),
            mcg_i, mul1_i, _stream(unpacked)))


def reconstruct_had_t(unpacked_t: Tensor, packed: Tensor, suh: Tensor, svh: Tensor,
                      K: float, mcg: bool = False, mul1: bool = False, n_offset: int = 0) -> None:
    """reconstruct_had_slice written transposed: unpacked_t (n, k) = (diag(suh) H W_hat H
    diag(svh))^T per 128 x 128 block, bit for bit the values of reconstruct_had_slice.  The
    layout recon_mm reads (no reference counterpart: the reference keeps W (k, n) for cuBLAS)."""
    bits, half = bits_from_K(K)
    _need(not half or mul1, "reconstruct: half-integer bitrates require the mul1 codebook")
    _need(packed.dim() == 3 and unpacked_t.dim() == 2, "reconstruct_had: bad tensor ranks")
    _need(unpacked_t.size(1) == packed.size(0) * 16 and n_offset >= 0
          and n_offset + unpacked_t.size(0) <= packed.size(1) * 16, "unpacked and packed shapes are incompatible")
    _need(packed.size(2) == 16 * bits + (8 if half else 0), "packed tile size does not match K")
    for t, nm in ((unpacked_t, "unpacked"), (suh, "suh"), (svh, "svh")):
        _dtype(t, torch.half, nm)
    _trellis_dtype(packed, "packed")
    if unpacked_t.numel() == 0:
        return
    _need(suh.numel() >= unpacked_t.size(1), "reconstruct_had: suh size")
    _need(svh.numel() >= unpacked_t.size(0), "reconstruct_had: svh size")
    _cuda(unpacked_t, packed, suh, svh)
    with torch.cuda.device(unpacked_t.device):
        check(_lib.lib().exl3_amd_reconstruct_had_t(
            unpacked_t.data_ptr(), packed.data_ptr(), suh.data_ptr(), svh.data_ptr(), unpacked_t.size(1),
            packed.size(1) * 16, unpacked_t.size(0), int(n_offset), float(K), int(bool(mcg)), int(bool(mul1)),
            _stream(unpacked_t)))


def _rows_k(t: Tensor) -> tuple:
    """(rows, k) of a recon operand: 2-D row-major (rows, k), or 3-D (k / 32, rows, 32) in the k-slab
    layout (slab c holds the 32 k from 32 c of every row)."""
    if t.dim() == 3:
        _need(t.size(2) == 32, "slab operand: last dimension must be 32")
        return t.size(1), t.size(0) * 32
    _need(t.dim() == 2, "recon operand must be 2-D (row-major) or 3-D (k slabs)")
    return t.size(0), t.size(1)


def slabs_of(t: Tensor) -> Tensor:
    """The k-slab form (k / 32, rows, 32) of a row-major (rows, k) tensor (a torch copy, for tests)."""
    return t.view(t.size(0), t.size(1) // 32, 32).transpose(0, 1).contiguous()


def recon_mm(a: Tensor, wt: Tensor, out: Tensor, svh: Optional[Tensor] = None) -> None:
    """out (m, n) = a (m, k) @ wt (n, k)^T on the hand-written MFMA kernel (exl3_amd_recon_mm),
    fp32 accumulation, out fp16 or fp32; with svh each 128-column chunk of the fp32 result is
    rotated (H128 / sqrt(128)) and scaled by svh before the store.  a and wt may each be given in
    the k-slab layout, (k / 32, rows, 32) (exl3_amd_recon_mm_slabs)."""
    _dtype(a, torch.half, "a")
    _dtype(wt, torch.half, "wt")
    _need(out.dtype in (torch.half, torch.float), "out is incorrect datatype, must be half or float")
    (m, k), (n, kw) = _rows_k(a), _rows_k(wt)
    _need(out.dim() == 2 and k == kw and out.shape == (m, n), "recon_mm: incompatible shapes")
    _need(a.is_contiguous() and wt.is_contiguous(), "recon_mm: tensors must be contiguous")
    # out may be a column block of a wider row-major tensor (rows ldc elements apart)
    _need(out.stride(1) == 1 and (m <= 1 or out.stride(0) >= n), "recon_mm: out rows must be contiguous")
    ldc = out.stride(0) if m > 1 else n
    if svh is not None:
        _dtype(svh, torch.half, "svh")
        _need(svh.numel() >= n, "svh too short")
    _cuda(a, wt, svh)
    _need(out.is_cuda, "tensors must be on a GPU device")
    with torch.cuda.device(a.device):
        if a.dim() == 2 and wt.dim() == 2 and ldc == n:
            check(_lib.lib().exl3_amd_recon_mm(a.data_ptr(), wt.data_ptr(), out.data_ptr(), int(out.dtype == torch.float),
                                               _ptr(svh), m, k, n, _stream(a)))
        else:
            check(_lib.lib().exl3_amd_recon_mm_slabs(a.data_ptr(), wt.data_ptr(), out.data_ptr(),
                                                     int(out.dtype == torch.float), _ptr(svh), m, k, n,
                                                     int(a.dim() == 3), int(wt.dim() == 3), ldc, _stream(a)))


def reconstruct_t_slabs(unpacked_s: Tensor, packed: Tensor, K: float, mcg: bool = False, mul1: bool = False,
                        suh: Optional[Tensor] = None, svh: Optional[Tensor] = None, n_offset: int = 0) -> None:
    """reconstruct_t (suh, svh None) or reconstruct_had_t (both given) written in the k-slab
    layout: unpacked_s (k / 32, n, 32) (exl3_amd_reconstruct_t_slabs)."""
    bits, half = bits_from_K(K)
    _need(not half or mul1, "reconstruct: half-integer bitrates require the mul1 codebook")
    _need(packed.dim() == 3 and unpacked_s.dim() == 3 and unpacked_s.size(2) == 32, "reconstruct_t_slabs: bad tensor ranks")
    n, k = unpacked_s.size(1), unpacked_s.size(0) * 32
    _need(k == packed.size(0) * 16 and n_offset >= 0 and n_offset + n <= packed.size(1) * 16,
          "unpacked and packed shapes are incompatible")
    _need(packed.size(2) == 16 * bits + (8 if half else 0), "packed tile size does not match K")
    _need((suh is None) == (svh is None), "reconstruct_t_slabs: give both suh and svh or neither")
    _dtype(unpacked_s, torch.half, "unpacked")
    _trellis_dtype(packed, "packed")
    if suh is not None:
        _dtype(suh, torch.half, "suh")
        _dtype(svh, torch.half, "svh")
        _need(suh.numel() >= k and svh.numel() >= n, "reconstruct_t_slabs: suh / svh size")
    if unpacked_s.numel() == 0:
        return
    _cuda(unpacked_s, packed, suh, svh)
    with torch.cuda.device(unpacked_s.device):
        check(_lib.lib().exl3_amd_reconstruct_t_slabs(
            unpacked_s.data_ptr(), packed.data_ptr(), _ptr(suh), _ptr(svh), k, packed.size(1) * 16, n,
            int(n_offset), float(K), int(bool(mcg)), int(bool(mul1)), int(suh is not None), _stream(unpacked_s)))


def to_slabs(x: Tensor, y: Tensor, rotate: bool = False, pre_scale: Optional[Tensor] = None,
             scale: float = 1.0) -> None:
    """y (k / 32, rows, 32) = x (rows, k) in the k-slab layout, copied or rotated like had_r_128
    (H128(x o pre_scale) * scale / sqrt(128)) on the way (exl3_amd_to_slabs)."""
    _dtype(x, torch.half, "x")
    _dtype(y, torch.half, "y")
    _need(x.dim() == 2 and y.dim() == 3 and y.shape == (x.size(1) // 32, x.size(0), 32) and x.size(1) % 32 == 0,
          "to_slabs: incompatible shapes")
    _need(x.is_contiguous() and y.is_contiguous(), "to_slabs: tensors must be contiguous")
    if pre_scale is not None:
        _dtype(pre_scale, torch.half, "pre_scale")
        _need(pre_scale.numel() >= x.size(1), "pre_scale too short")
    _cuda(x, y, pre_scale)
    with torch.cuda.device(x.device):
        check(_lib.lib().exl3_amd_to_slabs(x.data_ptr(), y.data_ptr(), x.size(0), x.size(1), int(bool(rotate)),
                                           _ptr(pre_scale), float(scale), _stream(x)))


def had_r_128(input: Tensor, output: Tensor, pre_scale: Optional[Tensor] = None,
              post_scale: Optional[Tensor] = None, scale: float = 1.0) -> None:
    """y = (x.view(-1, 128) @ H128 / sqrt(128)).view(x.shape) with an optional fp16 pre- or
    post-scale; works in place.  As in the reference, a given pre_scale takes precedence and
    post_scale is then ignored (hadamard.cu:170-186)."""
    _need(input.shape == output.shape, "input and output shapes differ")
    _need(input.dim() == 2, "input must be 2-dimensional")
    _need(input.size(1) % 128 == 0, "input columns must be divisible by 128")
    if input.dtype == torch.half:
        _dtype(output, torch.half, "output")
        fp32 = 0
    elif input.dtype == torch.float:
        _dtype(output, torch.float, "output")
        fp32 = 1
    else:
        raise _lib.Exl3Error(_lib.EINVAL, "unsupported datatype")
    if post_scale is not None and pre_scale is not None:
        post_scale = None
    for s in (pre_scale, post_scale):
        if s is not None:
            _dtype(s, torch.half, "scale")
            _need(s.numel() >= input.size(1), "scale vector too short")
    if input.numel() == 0:
        return
    _cuda(input, output, pre_scale, post_scale)
    with torch.cuda.device(input.device):
        check(_lib.lib().exl3_amd_had_r_128(
            input.data_ptr(), output.data_ptr(), input.size(0), input.size(1), fp32,
            _ptr(pre_scale), _ptr(post_scale), float(scale), _stream(input)))


def exl3_gemm(A: Tensor, B: Tensor, C: Tensor, suh: Optional[Tensor], A_had: Optional[Tensor],
              svh: Optional[Tensor], force_shape_idx: int = 0, mcg: bool = False,
              mul1: bool = False, force_num_sms: int = 0) -> int:
    """C = A @ dequant(B), with the input / output rotations when suh / svh are given.
    A (..., k) fp16, B trellis (k/16, n/16, 16K) int16, C (..., n) fp16 or fp32.
    Returns the kernel tag (90 = GEMV, 91 = MFMA GEMM).  force_num_sms is accepted for
    interface parity (the reference's cooperative-grid override) and has no effect."""
    _need(B.dim() == 3, "B must be 3-dimensional")
    _need(A.size(-1) == B.size(0) * 16, "A and B shapes are incompatible")
    _need(C.size(-1) == B.size(1) * 16, "C and B shapes are incompatible")
    _dtype(A, torch.half, "A")
    _trellis_dtype(B, "B")
    _need(C.dtype in (torch.half, torch.float), "C is incorrect datatype, must be half or float")
    tile = B.size(2)
    half_k = tile % 16 != 0
    _need(not half_k or (tile % 16 == 8 and mul1),
          "exl3_gemm: half-integer bitrates require the mul1 codebook")
    K = tile // 16 + (0.5 if half_k else 0.0)
    mcg_i, mul1_i = _codebook_flags(mcg, mul1)
    m = A.numel() // max(A.size(-1), 1) if A.size(-1) else 0
    _need(C.numel() == m * C.size(-1), "A and C row counts differ")
    _cuda(A, B, C, suh, svh)
    for s, n, name in ((suh, A.size(-1), "suh"), (svh, C.size(-1), "svh")):
        if s is not None:
            _dtype(s, torch.half, name)
            _need(s.numel() >= n, f"{name} too short")
    with torch.cuda.device(A.device):
        return check(_lib.lib().exl3_amd_gemm(
            A.data_ptr(), B.data_ptr(), C.data_ptr(), int(C.dtype == torch.float), _ptr(suh),
            _ptr(A_had), _ptr(svh), m, A.size(-1), C.size(-1), float(K), mcg_i, mul1_i,
            int(force_shape_idx), _stream(A)))


def exl3_mgemm(A: Tensor, B: Tensor, C: Tensor, suh: Tensor, A_had: Tensor, svh: Tensor,
               indices: Optional[Tensor], weights: Optional[Tensor], K: float,
               force_shape_idx: int = -1, mcg: int = 0, mul1: int = 0, min_index: int = -1,
               max_index: int = -1, force_num_sms: int = 0, num_tokens: int = 1,
               size_n_list: Optional[Tensor] = None, c_ptrs: Optional[Tensor] = None,
               n_stride_list: Optional[Tensor] = None, had_src_list: Optional[Tensor] = None,
               num_had_src: int = 0, norm_in: Optional[tuple] = None) -> int:
    """Multi-matrix EXL3 matmul over device pointer tables (exl3_gemm.cu:352-394 semantics).
    A (bszm_in, m, k) fp16; B / suh / svh int64 tensors of device addresses; C (bszm_out, m, n)
    fp16 or fp32; indices / weights (.., num_indices) int64 / fp16; optional int32 lists and
    int64 c_ptrs for per-matrix widths and sliced mode.  norm_in = (sq, w, eps, r): A is the
    residual stream h and the input is its split-norm form rmsnorm(h) * w, from the chunk sums
    sq (m, k / 128) fp32 (res_sq / exl3_gemm_res), with r (m, k) as scratch.  Returns the
    kernel tag."""
    _dtype(A, torch.half, "A")
    for t, name in ((B, "B"), (suh, "suh"), (svh, "svh")):
        _dtype(t, torch.long, name)
        _need(t.dim() == 1, f"{name} must be 1-dimensional")
    _need(A.dim() == 3 and C.dim() == 3, "A and C must be 3-dimensional")
    _need(A.size(1) == C.size(1), "A and C shapes are incompatible")
    _need(C.dtype in (torch.half, torch.float), "C is incorrect datatype, must be half or float")
    _cuda(A, B, C, suh, svh, A_had, indices, weights, size_n_list, c_ptrs, n_stride_list, had_src_list)
    num_indices = 0
    if indices is not None:
        _dtype(indices, torch.long, "indices")
        _need(indices.dim() == 2, "indices must be 2-dimensional")
        num_indices = indices.size(1)
    if weights is not None:
        _dtype(weights, torch.half, "weights")
        _need(weights.dim() == 2, "weights must be 2-dimensional")
    for t, name, dt in ((size_n_list, "size_n_list", torch.int32), (c_ptrs, "c_ptrs", torch.long),
                        (n_stride_list, "n_stride_list", torch.int32), (had_src_list, "had_src_list", torch.int32)):
        if t is not None:
            _dtype(t, dt, name)
    if norm_in is not None:
        sq, w, eps, r = norm_in
        _dtype(sq, torch.float, "sq")
        _dtype(w, torch.half, "w")
        _dtype(r, torch.half, "r")
        _need(indices is None and weights is None and num_tokens == 1 and min_index < 0,
              "mgemm norm_in: no indices, routing weights or token groups")
        _need(sq.numel() == A.size(1) * (A.size(2) // 128) and w.numel() == A.size(2)
              and r.numel() == A.size(1) * A.size(2), "mgemm norm_in: sq / w / r shapes")
        _cuda(sq, w, r)
        with torch.cuda.device(A.device):
            return check(_lib.lib().exl3_amd_mgemm_norm_in(
                A.data_ptr(), A.size(0), A.size(1), A.size(2),
                B.data_ptr(), B.size(0),
                C.data_ptr(), C.size(0), C.size(2), int(C.dtype == torch.float),
                suh.data_ptr(), suh.size(0),
                _ptr(A_had), A_had.numel() if A_had is not None else 0,
                svh.data_ptr(), svh.size(0),
                _ptr(size_n_list), _ptr(c_ptrs), c_ptrs.size(0) if c_ptrs is not None else 0,
                _ptr(n_stride_list), n_stride_list.size(0) if n_stride_list is not None else 0,
                _ptr(had_src_list), had_src_list.size(0) if had_src_list is not None else 0, int(num_had_src),
                float(K), int(bool(mcg)), int(bool(mul1)),
                sq.data_ptr(), w.data_ptr(), float(eps), r.data_ptr(),
                _stream(A)))
    with torch.cuda.device(A.device):
        return check(_lib.lib().exl3_amd_mgemm(
            A.data_ptr(), A.size(0), A.size(1), A.size(2),
            B.data_ptr(), B.size(0),
            C.data_ptr(), C.size(0), C.size(2), int(C.dtype == torch.float),
            suh.data_ptr(), suh.size(0),
            _ptr(A_had), A_had.numel() if A_had is not None else 0,
            svh.data_ptr(), svh.size(0),
            _ptr(indices), num_indices, _ptr(weights),
            float(K), int(force_shape_idx), int(bool(mcg)), int(bool(mul1)),
            int(min_index), int(max_index), int(force_num_sms), int(num_tokens),
            _ptr(size_n_list), _ptr(c_ptrs), c_ptrs.size(0) if c_ptrs is not None else 0,
            _ptr(n_stride_list), n_stride_list.size(0) if n_stride_list is not None else 0,
            _ptr(had_src_list), had_src_list.size(0) if had_src_list is not None else 0, int(num_had_src),
            _stream(A)))


def mgemm(x: Tensor, B_ptrs: Tensor, C: Tensor, suh_ptrs: Tensor, A_had: Tensor, svh_ptrs: Tensor,
          K: float, mcg: bool, mul1: bool, opts: Optional[dict] = None, norm_in: Optional[tuple] = None) -> Tensor:
    """torch.mgemm of the engine (amp_torch.cpp:10194-10330): stacked bundle (x broadcast,
    C (num, m, n)) or, with opts {size_n_list, c_ptrs, n_stride_list, had_src_list,
    num_had_src}, sliced mode.  norm_in: see exl3_mgemm.  Returns C."""
    o = opts or {}
    if opts is not None:
        for key in ("size_n_list", "c_ptrs", "n_stride_list", "had_src_list"):
            _need(o.get(key) is not None, f"mgemm: opts.{key} missing")
        _need(isinstance(o.get("num_had_src"), int), "mgemm: num_had_src missing")
    exl3_mgemm(x, B_ptrs, C, suh_ptrs, A_had, svh_ptrs, None, None, K, -1, int(mcg), int(mul1),
               -1, -1, 0, 1, o.get("size_n_list"), o.get("c_ptrs"), o.get("n_stride_list"),
               o.get("had_src_list"), int(o.get("num_had_src", 0)), norm_in=norm_in)
    return C


def ptr_array(tensors, device=None) -> Tensor:
    """int64 device tensor of data pointers (amp_torch.cpp:10333, torch.ptr_array)."""
    vals = [t if isinstance(t, int) else t.data_ptr() for t in tensors]
    return torch.tensor(vals, dtype=torch.long, device=device if device is not None else "cuda")


MOE_ACT = {"silu": 0, "gelu": 1, "relu2": 2, "silu_oai": 3}


def moe_coop_ctr_len(slots_max: int, bsz_max: int, I: int, Ho: int) -> int:
    """int32 scratch length of exl3_moe_coop (exl3_moe_coop.cuh:163-166)."""
    return slots_max * (I // 128) + bsz_max * (Ho // 128) + 2 + (slots_max + 1) + slots_max


def exl3_moe_coop(x: Tensor, sel: Tensor, rw: Tensor, min_expert: int, max_expert: int, Hi: int,
                  g_trellis: Tensor, g_suh: Tensor, g_svh: Tensor,
                  u_trellis: Tensor, u_suh: Tensor, u_svh: Tensor,
                  d_trellis: Tensor, d_suh: Tensor, d_svh: Tensor,
                  g_bias: Optional[Tensor], u_bias: Optional[Tensor], d_bias: Optional[Tensor],
                  Kg: float, Ku: float, Kd: float, mcg: bool, mul1: bool, act: int, act_limit: float,
                  gated: bool, had_g: Tensor, had_u: Tensor, gu_g: Tensor, gu_u: Tensor, act_out: Tensor,
                  d_out: Tensor, ctr: Tensor, out: Tensor, sh_out: Optional[Tensor] = None,
                  sh_gate_w: Optional[Tensor] = None, bits_g: Optional[Tensor] = None,
                  bits_u: Optional[Tensor] = None, bits_d: Optional[Tensor] = None) -> None:
    """Fused decode-shaped MoE, the tensor front end of exl3_moe_coop (exl3_moe_coop.cu:307-371):
    out (fp32, rows >= bsz) gets every token's routed experts summed with their routing weights
    (+ the shared expert).  Pointer tables are int64 device tensors indexed by local expert."""
    _dtype(x, torch.half, "x")
    _dtype(sel, torch.long, "sel")
    _dtype(rw, torch.half, "rw")
    _need(sel.is_contiguous() and rw.is_contiguous(), "exl3_moe_coop: sel/rw must be contiguous")
    _need(sel.shape == rw.shape and sel.dim() == 2 and sel.size(0) == x.size(0),
          "exl3_moe_coop: sel/rw must be (bsz, topk)")
    _need(x.dim() == 2 and x.stride(1) == 1, "exl3_moe_coop: x must be (bsz, H) with unit column stride")
    if sh_out is not None:
        _dtype(sh_out, torch.float, "sh_out")
        _need(sh_out.is_contiguous() and sh_out.size(-1) == x.size(1) and sh_out.numel() >= x.size(0) * x.size(1),
              "exl3_moe_coop: shared expert output shape")
    _dtype(ctr, torch.int32, "ctr")
    _need(ctr.is_contiguous(), "exl3_moe_coop: ctr must be contiguous")
    for t in (g_trellis, g_suh, g_svh, u_trellis, u_suh, u_svh, d_trellis, d_suh, d_svh):
        _need(t.dtype == torch.long and t.is_contiguous(), "exl3_moe_coop: pointer tables must be contiguous int64")
    for t, name in ((had_g, "had_g"), (had_u, "had_u"), (act_out, "act_out")):
        _dtype(t, torch.half, name)
    _dtype(d_out, torch.float, "d_out")
    _dtype(out, torch.float, "out")
    _need(gu_u.dtype in (torch.half, torch.float) and gu_g.dtype == gu_u.dtype,
          "exl3_moe_coop: gate/up scratch dtype mismatch")
    I, Ho = gu_u.size(-1), d_out.size(-1)
    for t, w in ((had_g, Hi), (had_u, Hi), (gu_g, I), (gu_u, I), (act_out, I), (d_out, Ho)):
        _need(t.is_contiguous() and t.size(-1) == w, "exl3_moe_coop: scratch shape")
    _need(out.dim() >= 2 and out.stride(-1) == 1, "exl3_moe_coop: out shape")
    if sh_gate_w is not None:
        _dtype(sh_gate_w, torch.half, "sh_gate_w")
        _need(sh_gate_w.is_contiguous(), "exl3_moe_coop: shared gate weight must be contiguous")
    bits = (bits_g, bits_u, bits_d)
    if any(b is not None for b in bits):
        _need(all(b is not None for b in bits), "exl3_moe_coop: give all three bit width tables or none")
        for b in bits:
            _need(b.dtype == torch.uint8 and b.is_contiguous() and b.numel() >= u_trellis.size(0),
                  "exl3_moe_coop: bit width tables must be contiguous uint8, one entry per expert")
    _cuda(x, sel, rw, ctr, out, had_g, had_u, act_out, d_out, gu_g, gu_u, sh_out, sh_gate_w, *bits)
    for b in (g_bias, u_bias, d_bias):
        if b is not None:
            _need(b.dtype == torch.long, "exl3_moe_coop: bias tables must be int64")
    with torch.cuda.device(x.device):
        check(_lib.lib().exl3_amd_moe_coop(
            x.data_ptr(), x.size(0), x.size(1), x.stride(0),
            sel.data_ptr(), rw.data_ptr(), sel.size(1),
            int(min_expert), int(max_expert), int(Hi),
            g_trellis.data_ptr(), g_suh.data_ptr(), g_svh.data_ptr(),
            u_trellis.data_ptr(), u_suh.data_ptr(), u_svh.data_ptr(),
            d_trellis.data_ptr(), d_suh.data_ptr(), d_svh.data_ptr(), u_trellis.size(0),
            _ptr(g_bias), _ptr(u_bias), _ptr(d_bias),
            float(Kg), float(Ku), float(Kd), int(bool(mcg)), int(bool(mul1)), int(act), float(act_limit),
            int(bool(gated)),
            had_g.data_ptr(), had_g.numel(), had_u.data_ptr(), had_u.numel(),
            gu_g.data_ptr(), gu_u.data_ptr(), min(gu_g.numel(), gu_u.numel()), int(gu_u.dtype == torch.float), I,
            act_out.data_ptr(), act_out.numel(), d_out.data_ptr(), d_out.numel(), Ho,
            ctr.data_ptr(), ctr.numel(),
            out.data_ptr(), out.size(-2), out.size(-1), out.stride(-2),
            _ptr(sh_out), _ptr(sh_gate_w), sh_gate_w.numel() if sh_gate_w is not None else 0,
            _ptr(bits_g), _ptr(bits_u), _ptr(bits_d),
            _stream(x)))


def exl3_moe_max_concurrency(device: int = 0) -> int:
    """exl3_moe_max_concurrency (exl3_moe.cu:15-19): the temp buffers' first dimension."""
    return check(_lib.lib().exl3_amd_moe_max_concurrency(int(device)))


def exl3_moe(hidden_state: Tensor, output_state: Tensor, expert_count: Tensor, token_sorted: Tensor,
             weight_sorted: Tensor, temp_state_g: Tensor, temp_state_u: Tensor,
             temp_intermediate_g: Tensor, temp_intermediate_u: Tensor, act_function: int,
             K_gate: float, K_up: float, K_down: float,
             gate_ptrs_trellis: Tensor, gate_ptrs_suh: Tensor, gate_ptrs_svh: Tensor,
             up_ptrs_trellis: Tensor, up_ptrs_suh: Tensor, up_ptrs_svh: Tensor,
             down_ptrs_trellis: Tensor, down_ptrs_suh: Tensor, down_ptrs_svh: Tensor,
             gate_mcg: bool, gate_mul1: bool, up_mcg: bool, up_mul1: bool, down_mcg: bool, down_mul1: bool,
             act_limit: float, num_active: int, output_scratch: Optional[Tensor] = None,
             fused_base: Optional[Tensor] = None, count_lo: int = 0, count_hi: int = 1 << 30,
             m_tile: int = 16, bits_g: Optional[Tensor] = None, bits_u: Optional[Tensor] = None,
             bits_d: Optional[Tensor] = None) -> None:
    """Token-sorted fused MoE, the tensor front end of exl3_moe (exl3_moe.cu:137-418): the experts
    with count_lo <= count <= count_hi (and count <= max_tokens_per_expert) run gate / up / act /
    down on their gathered rows and add weight * result into output_state (fp32, zeroed by the
    caller), or store it in their slots of output_scratch (then exl3_moe_gather sums in order)."""
    if num_active == 0:
        return
    if output_scratch is not None:
        _need(fused_base is not None, "exl3_moe: output_scratch needs fused_base")
        _dtype(output_scratch, torch.float, "output_scratch")
        _dtype(fused_base, torch.long, "fused_base")
        _need(output_scratch.is_contiguous() and output_scratch.dim() == 2
              and output_scratch.size(1) == hidden_state.size(1), "exl3_moe: output_scratch must be [slots, hidden]")
    _dtype(hidden_state, torch.half, "hidden_state")
    _need(hidden_state.dim() == 2 and hidden_state.is_contiguous(), "hidden_state must be 2-dimensional")
    _dtype(output_state, torch.float, "output_state")
    _need(output_state.shape == hidden_state.shape and output_state.is_contiguous(),
          "output_state and hidden_state shapes differ")
    _dtype(expert_count, torch.long, "expert_count")
    _need(expert_count.dim() == 1, "expert_count must be 1-dimensional")
    _dtype(token_sorted, torch.long, "token_sorted")
    _need(token_sorted.dim() == 1 and token_sorted.shape == weight_sorted.shape,
          "token_sorted and weight_sorted shapes differ")
    _dtype(weight_sorted, torch.half, "weight_sorted")
    for t, name in ((temp_state_g, "temp_state_g"), (temp_state_u, "temp_state_u"),
                    (temp_intermediate_g, "temp_intermediate_g"), (temp_intermediate_u, "temp_intermediate_u")):
        _dtype(t, torch.half, name)
        _need(t.dim() == 3 and t.is_contiguous(), f"{name} must be 3-dimensional")
    _need(temp_state_g.size(2) == hidden_state.size(1), "temp_state_g and hidden_state shapes differ")
    _need(temp_state_g.shape == temp_state_u.shape, "temp_state_g and temp_state_u shapes differ")
    _need(temp_intermediate_g.shape == temp_intermediate_u.shape, "temp_intermediate shapes differ")
    _need(temp_intermediate_g.size(1) == temp_state_g.size(1), "temp_intermediate_g and temp_state_g shapes differ")
    tables = (gate_ptrs_trellis, gate_ptrs_suh, gate_ptrs_svh, up_ptrs_trellis, up_ptrs_suh, up_ptrs_svh,
              down_ptrs_trellis, down_ptrs_suh, down_ptrs_svh)
    for t in tables:
        _need(t.dtype == torch.long and t.dim() == 1 and t.is_contiguous() and t.shape == gate_ptrs_trellis.shape,
              "exl3_moe: pointer tables must be contiguous int64 of one length")
    bits = (bits_g, bits_u, bits_d)
    if any(b is not None for b in bits):
        _need(all(b is not None for b in bits), "exl3_moe: give all three bit width tables or none")
        for b in bits:
            _need(b.dtype == torch.uint8 and b.is_contiguous() and b.numel() >= expert_count.numel() - 1,
                  "exl3_moe: bit width tables must be contiguous uint8, one entry per expert")
    _cuda(hidden_state, output_state, expert_count, token_sorted, weight_sorted, temp_state_g,
          temp_intermediate_g, output_scratch, fused_base, *bits)
    with torch.cuda.device(hidden_state.device):
        check(_lib.lib().exl3_amd_moe(
            hidden_state.data_ptr(), hidden_state.size(0), hidden_state.size(1), output_state.data_ptr(),
            expert_count.data_ptr(), expert_count.numel(), token_sorted.data_ptr(), weight_sorted.data_ptr(),
            token_sorted.numel(),
            temp_state_g.data_ptr(), temp_state_u.data_ptr(), temp_state_g.size(0), temp_state_g.size(1),
            temp_intermediate_g.data_ptr(), temp_intermediate_u.data_ptr(), temp_intermediate_g.size(2),
            int(act_function), float(K_gate), float(K_up), float(K_down),
            *[t.data_ptr() for t in tables], gate_ptrs_trellis.numel(),
            int(bool(gate_mcg)), int(bool(gate_mul1)), int(bool(up_mcg)), int(bool(up_mul1)),
            int(bool(down_mcg)), int(bool(down_mul1)),
            float(act_limit), int(num_active),
            _ptr(output_scratch), output_scratch.size(0) if output_scratch is not None else 0,
            output_scratch.size(1) if output_scratch is not None else 0, _ptr(fused_base),
            int(count_lo), int(count_hi), int(m_tile),
            _ptr(bits_g), _ptr(bits_u), _ptr(bits_d), bits_g.numel() if bits_g is not None else 0,
            _stream(hidden_state)))


def exl3_moe_gather(output_state: Tensor, output_scratch: Tensor, flat_expert: Tensor, inv_order: Tensor,
                    expert_start: Tensor, slot_base: Tensor, slot_kind: Tensor, weight_sorted: Tensor) -> None:
    """exl3_moe_gather (exl3_moe.cu:480-527): every token's top-k slots summed in k order into
    its fp32 output row."""
    _dtype(output_state, torch.float, "output_state")
    _dtype(output_scratch, torch.float, "output_scratch")
    for t, name in ((flat_expert, "flat_expert"), (inv_order, "inv_order"), (expert_start, "expert_start"),
                    (slot_base, "slot_base"), (slot_kind, "slot_kind")):
        _dtype(t, torch.long, name)
    _dtype(weight_sorted, torch.half, "weight_sorted")
    _need(output_state.is_contiguous() and output_state.dim() == 2, "exl3_moe_gather: output_state")
    _need(output_scratch.is_contiguous() and output_scratch.dim() == 2
          and output_scratch.size(1) == output_state.size(1), "exl3_moe_gather: output_scratch must be [slots, hidden]")
    _need(all(t.is_contiguous() for t in (flat_expert, inv_order, expert_start, slot_base, slot_kind, weight_sorted)),
          "exl3_moe_gather: index tensors must be contiguous")
    _cuda(output_state, output_scratch, flat_expert, inv_order, expert_start, slot_base, slot_kind, weight_sorted)
    with torch.cuda.device(output_state.device):
        check(_lib.lib().exl3_amd_moe_gather(
            output_state.data_ptr(), output_state.size(0), output_state.size(1),
            output_scratch.data_ptr(), output_scratch.size(1),
            flat_expert.data_ptr(), flat_expert.numel(), inv_order.data_ptr(),
            expert_start.data_ptr(), expert_start.numel(), slot_base.data_ptr(), slot_base.numel(),
            slot_kind.data_ptr(), slot_kind.numel(), weight_sorted.data_ptr(), _stream(output_state)))


def rms_norm_res(x: Tensor, r: Tensor, weight: Tensor, eps: float, y: Optional[Tensor] = None,
                 n: Optional[Tensor] = None):
    """Fused residual add + RMSNorm (amp_torch.cpp:10073-10160): returns [y, n] with
    y = x + r (fp16) and n = rmsnorm(y) * weight.  y / n are allocated unless given (a captured
    decode step passes persistent buffers; y may be x itself)."""
    for t, name in ((x, "x"), (r, "r"), (weight, "weight")):
        _dtype(t, torch.half, name)
    dim = weight.numel()
    _need(x.dim() >= 1 and r.dim() >= 1 and x.size(-1) == dim and r.size(-1) == dim and r.numel() == x.numel(),
          "rms_norm_res: weight/last-dim mismatch")
    _need(dim % 4 == 0, f"rms_norm_res: last dim ({dim}) must be a multiple of 4")
    y = torch.empty_like(x) if y is None else y
    n = torch.empty_like(x) if n is None else n
    _cuda(x, r, weight, y, n)
    with torch.cuda.device(x.device):
        check(_lib.lib().exl3_amd_rms_norm_res(x.data_ptr(), r.data_ptr(), weight.data_ptr(), y.data_ptr(),
                                               n.data_ptr(), x.numel() // max(dim, 1), dim, float(eps), _stream(x)))
    return [y, n]


def silu_mul(g: Tensor, u: Tensor, out: Optional[Tensor] = None) -> Tensor:
    """silu(g) * u elementwise in fp32, rounded to fp16 (amp_torch.cpp:4960-5005)."""
    _dtype(g, torch.half, "silu_mul: gate")
    _dtype(u, torch.half, "silu_mul: up")
    _need(g.numel() == u.numel(), "silu_mul: gate/up size mismatch")
    out = torch.empty_like(g) if out is None else out
    _cuda(g, u, out)
    with torch.cuda.device(g.device):
        check(_lib.lib().exl3_amd_silu_mul(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(), _stream(g)))
    return out


def exl3_gemm_silu_mul(gate: Tensor, up: Tensor, B: Tensor, C: Tensor, suh: Optional[Tensor],
                       svh: Optional[Tensor], mcg: bool = False, mul1: bool = False,
                       act: Optional[Tensor] = None, A_had: Optional[Tensor] = None) -> int:
    """C = exl3_gemm(silu_mul(gate, up)) (graphdec.uc:206-217) in one call; one launch at one
    row (the GEMV forms the SwiGLU product in its input load).  act / A_had: scratch of gate's
    shape (allocated when absent)."""
    _need(B.dim() == 3, "B must be 3-dimensional")
    _dtype(gate, torch.half, "gate")
    _dtype(up, torch.half, "up")
    _need(gate.shape == up.shape, "silu_mul: gate/up size mismatch")
    _need(gate.size(-1) == B.size(0) * 16, "A and B shapes are incompatible")
    _need(C.size(-1) == B.size(1) * 16, "C and B shapes are incompatible")
    _trellis_dtype(B, "B")
    _need(C.dtype in (torch.half, torch.float), "C is incorrect datatype, must be half or float")
    tile = B.size(2)
    half_k = tile % 16 != 0
    _need(not half_k or (tile % 16 == 8 and mul1), "exl3_gemm: half-integer bitrates require the mul1 codebook")
    K = tile // 16 + (0.5 if half_k else 0.0)
    mcg_i, mul1_i = _codebook_flags(mcg, mul1)
    act = torch.empty_like(gate) if act is None else act
    A_had = torch.empty_like(gate) if A_had is None else A_had
    m = gate.numel() // gate.size(-1)
    _cuda(gate, up, act, B, C, suh, svh, A_had)
    with torch.cuda.device(gate.device):
        return check(_lib.lib().exl3_amd_gemm_silu_mul(
            gate.data_ptr(), up.data_ptr(), act.data_ptr(), B.data_ptr(), C.data_ptr(), int(C.dtype == torch.float),
            _ptr(suh), A_had.data_ptr(), _ptr(svh), m, gate.size(-1), C.size(-1), float(K), mcg_i, mul1_i,
            _stream(gate)))


def exl3_gemm_norm(A: Tensor, B: Tensor, C: Tensor, suh: Optional[Tensor], svh: Optional[Tensor],
                   h: Tensor, weight: Tensor, r: Tensor, eps: float, mcg: bool = False, mul1: bool = False,
                   up: Optional[Tensor] = None, act: Optional[Tensor] = None, A_had: Optional[Tensor] = None) -> int:
    """C = exl3_gemm(A) (of silu(A) * up when up is given), then [h, r] = rms_norm_res(h, C,
    weight) with h updated in place: one launch at one row (the GEMV's last chunk normalises)."""
    _need(B.dim() == 3, "B must be 3-dimensional")
    _dtype(A, torch.half, "A")
    _trellis_dtype(B, "B")
    _dtype(C, torch.half, "C")
    for t, nm in ((h, "h"), (weight, "weight"), (r, "r")):
        _dtype(t, torch.half, nm)
    k, n = B.size(0) * 16, B.size(1) * 16
    _need(A.size(-1) == k and C.size(-1) == n and h.numel() == C.numel() and r.numel() == C.numel()
          and weight.numel() == n, "exl3_gemm_norm: incompatible shapes")
    if up is not None:
        _dtype(up, torch.half, "up")
        _need(up.shape == A.shape, "silu_mul: gate/up size mismatch")
    tile = B.size(2)
    half_k = tile % 16 != 0
    _need(not half_k or (tile % 16 == 8 and mul1), "exl3_gemm: half-integer bitrates require the mul1 codebook")
    K = tile // 16 + (0.5 if half_k else 0.0)
    mcg_i, mul1_i = _codebook_flags(mcg, mul1)
    act = torch.empty_like(A) if (act is None and up is not None) else act
    A_had = torch.empty_like(A) if A_had is None else A_had
    m = A.numel() // k
    _cuda(A, B, C, suh, svh, h, weight, r, up, act, A_had)
    with torch.cuda.device(A.device):
        return check(_lib.lib().exl3_amd_gemm_norm(
            A.data_ptr(), _ptr(up), _ptr(act), B.data_ptr(), C.data_ptr(), _ptr(suh), A_had.data_ptr(), _ptr(svh),
            m, k, n, float(K), mcg_i, mul1_i, h.data_ptr(), weight.data_ptr(), r.data_ptr(), float(eps),
            _stream(A)))


def res_sq(h: Tensor, c: Optional[Tensor], sq: Tensor) -> None:
    """Producer half of the split residual norm on its own: h = fp16(h + c) in place (c None:
    h unchanged) and sq (rows, n / 128) fp32 = each 128-column chunk's sum of squares."""
    _dtype(h, torch.half, "h")
    _dtype(sq, torch.float, "sq")
    n = h.size(-1)
    rows = h.numel() // max(n, 1)
    _need(n % 128 == 0 and sq.numel() == rows * (n // 128), "res_sq: h / sq shapes")
    if c is not None:
        _dtype(c, torch.half, "c")
        _need(c.numel() == h.numel(), "res_sq: h / c shapes")
    _cuda(h, c, sq)
    with torch.cuda.device(h.device):
        check(_lib.lib().exl3_amd_res_sq(h.data_ptr(), _ptr(c), sq.data_ptr(), rows, n, _stream(h)))


def norm_sq(h: Tensor, sq: Tensor, weight: Tensor, eps: float, r: Optional[Tensor] = None) -> Tensor:
    """Consumer half of the split residual norm on its own: r = fp16(fp16(h * scale) * weight),
    scale = 1 / sqrt(sum(sq) / n + eps) from the chunk sums.  Returns r."""
    _dtype(h, torch.half, "h")
    _dtype(sq, torch.float, "sq")
    _dtype(weight, torch.half, "weight")
    n = h.size(-1)
    rows = h.numel() // max(n, 1)
    _need(n % 128 == 0 and sq.numel() == rows * (n // 128) and weight.numel() == n, "norm_sq: shapes")
    r = torch.empty_like(h) if r is None else r
    _cuda(h, sq, weight, r)
    with torch.cuda.device(h.device):
        check(_lib.lib().exl3_amd_norm_sq(h.data_ptr(), sq.data_ptr(), weight.data_ptr(), r.data_ptr(), rows, n,
                                          float(eps), _stream(h)))
    return r


def exl3_gemm_res(A: Tensor, B: Tensor, C: Tensor, suh: Optional[Tensor], svh: Optional[Tensor],
                  h: Tensor, sq: Tensor, mcg: bool = False, mul1: bool = False,
                  up: Optional[Tensor] = None, act: Optional[Tensor] = None, A_had: Optional[Tensor] = None) -> int:
    """C = exl3_gemm(A) (of silu(A) * up when up is given), then the producer half of the split
    residual norm: h = fp16(h + C) in place, sq = its chunk sums of squares.  One launch at one
    row (the GEMV's chunk epilogue)."""
    _need(B.dim() == 3, "B must be 3-dimensional")
    _dtype(A, torch.half, "A")
    _trellis_dtype(B, "B")
    _dtype(C, torch.half, "C")
    _dtype(h, torch.half, "h")
    _dtype(sq, torch.float, "sq")
    k, n = B.size(0) * 16, B.size(1) * 16
    m = A.numel() // k
    _need(A.size(-1) == k and C.size(-1) == n and h.numel() == C.numel() and sq.numel() == m * (n // 128),
          "exl3_gemm_res: incompatible shapes")
    if up is not None:
        _dtype(up, torch.half, "up")
        _need(up.shape == A.shape, "silu_mul: gate/up size mismatch")
    tile = B.size(2)
    half_k = tile % 16 != 0
    _need(not half_k or (tile % 16 == 8 and mul1), "exl3_gemm: half-integer bitrates require the mul1 codebook")
    K = tile // 16 + (0.5 if half_k else 0.0)
    mcg_i, mul1_i = _codebook_flags(mcg, mul1)
    act = torch.empty_like(A) if (act is None and up is not None) else act
    A_had = torch.empty_like(A) if A_had is None else A_had
    _cuda(A, B, C, suh, svh, h, sq, up, act, A_had)
    with torch.cuda.device(A.device):
        return check(_lib.lib().exl3_amd_gemm_res(
            A.data_ptr(), _ptr(up), _ptr(act), B.data_ptr(), C.data_ptr(), _ptr(suh), A_had.data_ptr(), _ptr(svh),
            m, k, n, float(K), mcg_i, mul1_i, h.data_ptr(), sq.data_ptr(), _stream(A)))


def _library_mm(a: Tensor, b: Tensor, out: Tensor) -> None:
    """out = a @ b on the vendor GEMM library (hipBLASLt / rocBLAS through torch.mm, TunableOp
    scoped to this call): the comparison path of bench.py, never the default route."""
    tun = getattr(torch.cuda, "tunable", None)
    if tun is None:
        torch.mm(a, b, out=out)
        return
    was = tun.is_enabled()
    if not was:
        tun.enable(True)
    try:
        torch.mm(a, b, out=out)
    finally:
        if not was:
            tun.enable(False)


def _recon_slabs(x: Tensor, y: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor, K: float, mcg: bool,
                 mul1: bool, fused: bool, k: int, n: int, rows: int) -> None:
    """exl3_gemm_recon's slab route: the x operand in k slabs (rotated, a copy, or x itself), the
    weight reconstructed in k slabs, one recon_mm_slabs.  (Measured and not kept: the x pass on a
    side stream beside the reconstruction, 1 % slower; the weight in 2-8 column chunks whose GEMMs
    start on side streams as their chunks are written, 1-2 % faster at 2 chunks and up to 2x
    slower at 4-8, where the chunks' GEMMs do not run side by side.)"""
    if fused and n < RECON_FUSED_X_SLABS_MIN_N:
        xa = x
    else:
        xa = torch.empty((k // 32, rows, 32), dtype=x.dtype, device=x.device)
        if fused:
            to_slabs(x, xa)
        else:
            to_slabs(x, xa, True, suh, 1.0)
    wt = torch.empty((k // 32, n, 32), dtype=x.dtype, device=x.device)
    if fused:
        reconstruct_t_slabs(wt, trellis, K, mcg, mul1, suh, svh)
    else:
        reconstruct_t_slabs(wt, trellis, K, mcg, mul1)
    recon_mm(xa, wt, y, None if fused else svh)


def exl3_gemm_recon(x: Tensor, trellis: Tensor, suh: Tensor, svh: Tensor, K: float,
                    mul1: bool = False, mcg: bool = False, fused_rows: Optional[int] = None,
                    gemm: str = "hip", slabs: bool = True) -> Tensor:
    """The reference's many-rows policy (amp_torch.cpp:11149-11230): reconstruct the weight to
    fp16 once, then one dense GEMM.  rows >= 2048: original-basis W and y = x @ W; otherwise
    y = had(had(x o suh) @ W_hat) o svh.  The weight is reconstructed transposed, and the dense
    GEMM is this build's MFMA kernel (recon_mm), which in the rotated branch also applies the
    output rotation and svh in its epilogue.  With slabs (the default) the reconstructed weight
    and the GEMM's activation operand are written in the k-slab layout, which the GEMM streams
    faster (x itself is copied into slabs for wide weights, RECON_FUSED_X_SLABS_MIN_N); slabs=False keeps both
    row-major (same results bit for bit).  gemm="library" runs the same reconstructions with the
    vendor GEMM (torch.mm) instead, for comparison."""
    _need(trellis.dim() == 3, "exl3_gemm_recon: trellis must be 3-D")
    _need(gemm in ("hip", "library"), "exl3_gemm_recon: gemm must be 'hip' or 'library'")
    k, n = trellis.size(0) * 16, trellis.size(1) * 16
    _need(x.dim() == 2 and x.size(1) == k and suh.numel() == k and svh.numel() == n and n <= 32768,
          f"exl3_gemm_recon: incompatible shapes (x {tuple(x.shape)}, weight {k} x {n})")
    rows = x.size(0)
    y = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    slabs = slabs and gemm == "hip" and k % 32 == 0
    fused = rows >= (RECON_FUSED_ROWS if fused_rows is None else fused_rows)
    if slabs:
        _recon_slabs(x.contiguous(), y, trellis, suh, svh, K, mcg, mul1, fused, k, n, rows)
        return y
    wt = torch.empty((n, k), dtype=x.dtype, device=x.device)
    if fused:
        reconstruct_had_t(wt, trellis, suh, svh, K, mcg, mul1, 0)
        if gemm == "hip":
            recon_mm(x.contiguous(), wt, y)
        else:
            _library_mm(x, wt.t(), y)
    else:
        xh = torch.empty_like(x)
        had_r_128(x, xh, suh, None, 1.0)
        reconstruct_t(wt, trellis, K, mcg, mul1)
        if gemm == "hip":
            recon_mm(xh, wt, y, svh)
        else:
            _library_mm(xh, wt.t(), y)
            had_r_128(y, y, None, svh, 1.0)
    return y


def init(device: int = 0) -> None:
    """Allocate the per-device workspace now (before graph capture)."""
    check(_lib.lib().exl3_amd_init(int(device)))
