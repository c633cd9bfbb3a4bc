"""fp16 products with an fp32 result split along the contraction (cm_gemm_f32), for the narrow,
long-contraction products of the training step's MLP (the down projection's forward and the
input gradient dgate Wg + dup Wu): C = A0 B0^T (+ A1 B1^T), deterministic; with b_kmajor the
B operands are given as [K, N] (C = A0 B0 + A1 B1: weights as stored, cm_gemm_f32_kb)."""

import torch

from . import _lib


def _operand(t):
    if t.dtype != torch.float16 or t.dim() != 2 or t.stride(1) != 1 or t.stride(0) % 8:
        return None
    if t.data_ptr() % 16 or t.shape[1] % 8:
        return None
    return t


def split_k_pays(m, n, k):
    """Whether an fp32-output product is better split along k: its output alone gives under
    half of the CUs a 256 x 192 tile, and the contraction is long (the MLP's down projection
    and input gradient at a few thousand tokens: hipBLASLt 55-69 us, split 43 us + 6 us sum)."""
    tiles = -(-m // 256) * -(-n // 192)
    return tiles < 128 and k >= 4096


def gemm_f32_supported(m, n, *pairs, b_kmajor=False):
    """Whether cm_gemm_f32 takes these operands: fp16, row-major with 16-byte aligned rows,
    contractions multiples of 8, on the GPU, and an output of a multiple of 4 elements (with
    b_kmajor, B [K, N] with N a multiple of 8)."""
    if not pairs or len(pairs) > 2 or (m * n) % 4:
        return False
    dev = pairs[0][0].device
    for a, b in pairs:
        if _operand(a) is None or _operand(b) is None:
            return False
        if not (a.is_cuda and b.is_cuda and a.device == dev and b.device == dev):
            return False
        if b_kmajor:
            if a.shape[0] != m or b.shape[1] != n or a.shape[1] != b.shape[0]:
                return False
        elif a.shape[0] != m or b.shape[0] != n or a.shape[1] != b.shape[1]:
            return False
    return True


def gemm_f32(*pairs, out=None, residual=None, b_kmajor=False):
    """sum over the (A [M, K], B [N, K]) pairs of A @ B^T, fp32 [M, N]; with `residual` (fp32 [M, N]
    contiguous) residual + that sum, added in the same launch (cm_gemm_f32_add); with b_kmajor
    the pairs are (A [M, K], B [K, N]) and the sum is of A @ B (cm_gemm_f32_kb)."""
    (a0, b0), rest = pairs[0], pairs[1:]
    m, n = a0.shape[0], (b0.shape[1] if b_kmajor else b0.shape[0])
    if out is None:
        out = torch.empty(m, n, dtype=torch.float32, device=a0.device)
    if m == 0 or n == 0:
        return out
    k0 = a0.shape[1]
    a1, b1 = rest[0] if rest else (None, None)
    k1 = a1.shape[1] if rest else 0
    ws_bytes = int(_lib.load().cm_gemm_f32_workspace_bytes(m, n, k0, k1))
    if ws_bytes < 0:
        raise RuntimeError("cm_gemm_f32_workspace_bytes: invalid shape")
    ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=a0.device)
    common = (a0.data_ptr(), a0.stride(0), b0.data_ptr(), b0.stride(0), k0, _lib.ptr(a1),
              a1.stride(0) if rest else 0, _lib.ptr(b1), b1.stride(0) if rest else 0, k1, m, n)
    if b_kmajor:
        if residual is not None:
            raise ValueError("gemm_f32: a residual is not taken with k-major B operands")
        _lib.call("cm_gemm_f32_kb", *common, out.data_ptr(), ws.data_ptr(), ws_bytes,
                  _lib.stream(a0.device))
    elif residual is None:
        _lib.call("cm_gemm_f32", *common, out.data_ptr(), ws.data_ptr(), ws_bytes,
                  _lib.stream(a0.device))
    else:
        if (residual.dtype != torch.float32 or residual.shape != (m, n)
                or not residual.is_contiguous()):
            raise ValueError("gemm_f32: the residual must be a contiguous fp32 [M, N] tensor")
        _lib.call("cm_gemm_f32_add", *common, residual.data_ptr(), out.data_ptr(),
                  ws.data_ptr(), ws_bytes, _lib.stream(a0.device))
    return out
