"""Device operators of the W4A16 hot path (PyTorch-ROCm tensors in, HIP kernels run).

Functional layer over the C ABI (``include/t2i_hip.h``).  Tensors must be CUDA
(HIP) tensors; every call launches on torch's current stream and returns
without synchronising.  Argument errors raise ``ValueError`` and HIP errors
``RuntimeError``, as the reference's operators do.
"""

from __future__ import annotations

import torch

from torch2iron_amd import _lib
from torch2iron_amd.formats import GROUP_SIZE, W4A16Weight

BF16 = torch.bfloat16

ROPE_HALVES = 0
PROMPT_GEMM_ROWS = 512   # rows from which the linear runs the LDS-tiled prompt GEMM (t2i_w4a16_linear)
ROPE_INTERLEAVED = 1


class Workspace:
    """Device scratch buffers keyed by purpose (the split-context attention's
    per-split partial results).  A buffer must not be used by two launches
    that overlap in time."""

    def __init__(self):
        self._bufs: dict = {}

    def get(self, key, nbytes: int, device) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        k = (key, torch.device(device))
        buf = self._bufs.get(k)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            self._bufs[k] = buf
        return buf


DEFAULT_WORKSPACE = Workspace()


def _check_dev(name: str, t: torch.Tensor, dtype=None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the W4A16 path has no CPU fallback)")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_sums(name: str, t: torch.Tensor, rows: int, per_row: int):
    """fp32 row group sums, group-major ``[per_row, rows]`` (see ``rmsnorm(out_sums=...)``)."""
    _check_dev(name, t, torch.float32)
    if t.numel() != rows * per_row:
        raise ValueError(f"{name} must hold {rows}x{per_row} sums")


def _check_weight(w: W4A16Weight):
    if not isinstance(w, W4A16Weight):
        raise ValueError("weight must be a W4A16Weight")
    for n, t in (("qweight", w.qweight), ("qzeros", w.qzeros), ("scales", w.scales)):
        _check_dev(n, t)


def dequantize(w: W4A16Weight) -> torch.Tensor:
    """Exact fp32 ``W [N, K]`` on the device (test hook for bit-exact parity)."""
    _check_weight(w)
    lib = _lib.load()
    out = torch.empty(w.N, w.K, dtype=torch.float32, device=w.qweight.device)
    rc = lib.t2i_w4a16_dequant_f32(w.qweight.data_ptr(), w.qzeros.data_ptr(), w.scales.data_ptr(),
                                   w.K, w.N, w.group_size, out.data_ptr(), _lib.stream_handle(out.device))
    _lib.check(rc, "t2i_w4a16_dequant_f32")
    return out


def tile_weight(w: W4A16Weight) -> W4A16Weight:
    """Give ``w`` its decode-linear tiles (``w.tiles``): qweight's words regrouped so
    that each workgroup of the decode linear reads whole, contiguous lines (a
    permutation, see ``t2i_w4a16_tile_qweight``).  From then on the linears below
    (without handed-over row sums) go through ``t2i_w4a16_linear_tiles``, which
    reads the tiles for the decode plans that gain from them and qweight for the
    rest and for prompt rows: bit-identical results.  Returns ``w``."""
    _check_weight(w)
    if w.tiles is None:
        tiles = torch.empty(w.qweight.numel(), dtype=torch.int32, device=w.qweight.device)
        lib = _lib.load()
        rc = lib.t2i_w4a16_tile_qweight(w.qweight.data_ptr(), w.K, w.N, tiles.data_ptr(),
                                        _lib.stream_handle(tiles.device))
        _lib.check(rc, "t2i_w4a16_tile_qweight")
        w.tiles = tiles
    return w


def _tiles_for(w: W4A16Weight):
    """The weight's tiles, checked, or None."""
    if w.tiles is None:
        return None
    _check_dev("tiles", w.tiles, torch.int32)
    if w.tiles.numel() != w.qweight.numel():
        raise ValueError("tiles must hold as many words as qweight")
    return w.tiles


def _linear_tiles(x2, m, norm_weight, eps, tiles, w, epilogue, residual, out, out_up, name):
    lib = _lib.load()
    rc = lib.t2i_w4a16_linear_tiles(x2.data_ptr(), m, _lib.ptr(norm_weight), float(eps), w.qweight.data_ptr(),
                                    tiles.data_ptr(), w.qzeros.data_ptr(), w.scales.data_ptr(), w.K, w.N,
                                    w.group_size, epilogue, _lib.ptr(residual), out.data_ptr(), _lib.ptr(out_up),
                                    _lib.stream_handle(x2.device))
    _lib.check(rc, f"t2i_w4a16_linear_tiles ({name})")


def linear(x: torch.Tensor, w: W4A16Weight, residual: torch.Tensor | None = None,
           out: torch.Tensor | None = None, x_sums: torch.Tensor | None = None,
           sum_parts: int = 1) -> torch.Tensor:
    """``y = x @ W^T`` (+ residual, rounded as bf16(bf16(x W^T) + residual)).

    ``x`` bf16 ``[M, K]`` (or ``[K]`` for the GEMV case): M = 1 is the GEMV,
    M <= 64 a decode batch, more rows a prompt batch.  ``x_sums``: fp32 sums of
    each row of ``x`` over each 128-wide k group (``sum_parts=1``, group-major
    ``[K/128, M]``) or 64-wide half group (``sum_parts=2``, ``[K/64, M]``), as the
    kernel that wrote ``x`` emits them; the prompt GEMM then skips forming them.
    """
    _check_weight(w)
    _check_dev("x", x, BF16)
    squeeze = x.dim() == 1
    x2 = x.view(1, -1) if squeeze else x
    if x2.dim() != 2 or x2.shape[1] != w.K:
        raise ValueError(f"x shape {tuple(x.shape)} does not match K={w.K}")
    m = x2.shape[0]
    if out is None:
        out = torch.empty(m, w.N, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * w.N:
        raise ValueError(f"out must hold {m}x{w.N} elements")
    if residual is not None:
        _check_dev("residual", residual, BF16)
        if residual.numel() != m * w.N:
            raise ValueError(f"residual must hold {m}x{w.N} elements")
    lib = _lib.load()
    tiles = _tiles_for(w) if x_sums is None else None
    if tiles is not None:
        _linear_tiles(x2, m, None, 0.0, tiles, w, _lib.T2I_TILES_STORE, residual, out, None, "linear")
    elif x_sums is not None:
        _check_sums("x_sums", x_sums, m, sum_parts * (w.K // w.group_size))
        rc = lib.t2i_w4a16_linear_sums(x2.data_ptr(), x_sums.data_ptr(), int(sum_parts), m, w.qweight.data_ptr(),
                                       w.qzeros.data_ptr(), w.scales.data_ptr(), w.K, w.N, w.group_size,
                                       _lib.ptr(residual), out.data_ptr(), _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_linear_sums")
    else:
        rc = lib.t2i_w4a16_linear(x2.data_ptr(), m, w.qweight.data_ptr(), w.qzeros.data_ptr(), w.scales.data_ptr(),
                                  w.K, w.N, w.group_size, _lib.ptr(residual), out.data_ptr(),
                                  _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_linear")
    return out.view(-1) if squeeze else out.view(m, w.N)


def gate_up(x: torch.Tensor, w_pair: W4A16Weight, swiglu: bool = True, out: torch.Tensor | None = None,
            out_up: torch.Tensor | None = None, x_sums: torch.Tensor | None = None, sum_parts: int = 1,
            out_sums: torch.Tensor | None = None):
    """Paired gate/up projection over an ``interleave_gate_up`` weight.

    ``swiglu=True``: returns ``h = silu(gate) * up`` bf16 ``[M, N/2]``.
    ``swiglu=False``: returns ``(gate, up)``, each ``[M, N/2]``.
    ``x_sums`` / ``sum_parts`` as ``linear``.  ``out_sums`` (SwiGLU, prompt rows
    only): fp32 ``[N/128, M]`` receives each row of ``h`` summed over its 64-wide
    half groups, the down projection's ``x_sums`` with ``sum_parts=2``.
    """
    _check_weight(w_pair)
    _check_dev("x", x, BF16)
    x2 = x.view(1, -1) if x.dim() == 1 else x
    if x2.dim() != 2 or x2.shape[1] != w_pair.K:
        raise ValueError(f"x shape {tuple(x.shape)} does not match K={w_pair.K}")
    m, inter = x2.shape[0], w_pair.N // 2
    if out is None:
        out = torch.empty(m, inter, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * inter:
        raise ValueError(f"out must hold {m}x{inter} elements")
    if not swiglu:
        if out_up is None:
            out_up = torch.empty(m, inter, dtype=BF16, device=x.device)
        _check_dev("out_up", out_up, BF16)
        if out_up.numel() != m * inter:
            raise ValueError(f"out_up must hold {m}x{inter} elements")
    lib = _lib.load()
    tiles = _tiles_for(w_pair) if x_sums is None and out_sums is None else None
    if tiles is not None:
        _linear_tiles(x2, m, None, 0.0, tiles, w_pair, _lib.T2I_TILES_SWIGLU if swiglu else _lib.T2I_TILES_PAIRED,
                      None, out, out_up, "gate_up")
    elif x_sums is not None or out_sums is not None:
        if x_sums is not None:
            _check_sums("x_sums", x_sums, m, sum_parts * (w_pair.K // w_pair.group_size))
        if out_sums is not None:
            _check_sums("out_sums", out_sums, m, w_pair.N // 128)
        rc = lib.t2i_w4a16_gate_up_sums(x2.data_ptr(), _lib.ptr(x_sums), int(sum_parts), m,
                                        w_pair.qweight.data_ptr(), w_pair.qzeros.data_ptr(), w_pair.scales.data_ptr(),
                                        w_pair.K, w_pair.N, w_pair.group_size, int(bool(swiglu)), out.data_ptr(),
                                        _lib.ptr(out_up), _lib.ptr(out_sums), _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_gate_up_sums")
    else:
        rc = lib.t2i_w4a16_gate_up(x2.data_ptr(), m, w_pair.qweight.data_ptr(), w_pair.qzeros.data_ptr(),
                                   w_pair.scales.data_ptr(), w_pair.K, w_pair.N, w_pair.group_size,
                                   int(bool(swiglu)), out.data_ptr(), _lib.ptr(out_up), _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_gate_up")
    return out if swiglu else (out, out_up)


def rmsnorm_linear(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w: W4A16Weight,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """``y = rmsnorm(x) @ W^T`` with the RMSNorm done inside the linear kernel
    (``x`` bf16 ``[M, K]`` is the un-normalised residual stream, 1 <= M <= 64): the
    kernel multiplies ``bf16(x * norm_weight)`` and scales each row's sums by its
    ``1 / rms``, so it equals the unfused pair up to where products round to bf16."""
    _check_weight(w)
    _check_dev("x", x, BF16)
    _check_dev("norm_weight", norm_weight, BF16)
    x2 = x.view(1, -1) if x.dim() == 1 else x
    if x2.dim() != 2 or x2.shape[1] != w.K or norm_weight.numel() != w.K:
        raise ValueError(f"x shape {tuple(x.shape)} / norm_weight do not match K={w.K}")
    m = x2.shape[0]
    if out is None:
        out = torch.empty(m, w.N, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * w.N:
        raise ValueError(f"out must hold {m}x{w.N} elements")
    tiles = _tiles_for(w)
    if tiles is not None:
        _linear_tiles(x2, m, norm_weight, eps, tiles, w, _lib.T2I_TILES_STORE, None, out, None, "rmsnorm_linear")
    else:
        lib = _lib.load()
        rc = lib.t2i_w4a16_rmsnorm_linear(x2.data_ptr(), m, norm_weight.data_ptr(), float(eps), w.qweight.data_ptr(),
                                          w.qzeros.data_ptr(), w.scales.data_ptr(), w.K, w.N, w.group_size,
                                          out.data_ptr(), _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_rmsnorm_linear")
    return out.view(m, w.N) if x.dim() != 1 else out.view(-1)


def rmsnorm_gate_up(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, w_pair: W4A16Weight,
                    swiglu: bool = True, out: torch.Tensor | None = None, out_up: torch.Tensor | None = None):
    """RMSNorm fused into the paired gate/up projection (see ``gate_up``)."""
    _check_weight(w_pair)
    _check_dev("x", x, BF16)
    _check_dev("norm_weight", norm_weight, BF16)
    x2 = x.view(1, -1) if x.dim() == 1 else x
    if x2.dim() != 2 or x2.shape[1] != w_pair.K or norm_weight.numel() != w_pair.K:
        raise ValueError(f"x shape {tuple(x.shape)} / norm_weight do not match K={w_pair.K}")
    m, inter = x2.shape[0], w_pair.N // 2
    if out is None:
        out = torch.empty(m, inter, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * inter:
        raise ValueError(f"out must hold {m}x{inter} elements")
    if not swiglu:
        if out_up is None:
            out_up = torch.empty(m, inter, dtype=BF16, device=x.device)
        _check_dev("out_up", out_up, BF16)
        if out_up.numel() != m * inter:
            raise ValueError(f"out_up must hold {m}x{inter} elements")
    tiles = _tiles_for(w_pair)
    if tiles is not None:
        _linear_tiles(x2, m, norm_weight, eps, tiles, w_pair,
                      _lib.T2I_TILES_SWIGLU if swiglu else _lib.T2I_TILES_PAIRED, None, out, out_up,
                      "rmsnorm_gate_up")
    else:
        lib = _lib.load()
        rc = lib.t2i_w4a16_rmsnorm_gate_up(x2.data_ptr(), m, norm_weight.data_ptr(), float(eps),
                                           w_pair.qweight.data_ptr(), w_pair.qzeros.data_ptr(),
                                           w_pair.scales.data_ptr(), w_pair.K, w_pair.N, w_pair.group_size,
                                           int(bool(swiglu)), out.data_ptr(), _lib.ptr(out_up),
                                           _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_w4a16_rmsnorm_gate_up")
    return out if swiglu else (out, out_up)


# ---- chained RMSNorm between decode linears (over tiles) ----
CHAIN_PRODUCER, CHAIN_CONSUMER, CHAIN_PAIRED_CONSUMER = 0, 1, 2


def chain_supported(m: int, k: int, n: int, role: int) -> bool:
    """Whether a decode linear of ``m`` rows, K = ``k``, N = ``n`` has a chained-norm
    form in ``role`` (``CHAIN_PRODUCER``: residual epilogue that also writes the next
    norm's input; ``CHAIN_CONSUMER`` / ``CHAIN_PAIRED_CONSUMER``: the fused-norm linear /
    gate_up taking that input)."""
    return bool(_lib.load().t2i_w4a16_chain_supported(int(m), int(k), int(n), int(role)))


def _chain_call(name, x2, m, ss_in, eps, w, epilogue, residual, out, out_up, next_norm, xg_out, ss_out):
    tiles = _tiles_for(w)
    if tiles is None:
        raise ValueError("the chained norm reads the weight's tiles: call tile_weight first")
    lib = _lib.load()
    rc = lib.t2i_w4a16_linear_tiles_chain(x2.data_ptr(), m, _lib.ptr(ss_in), float(eps), w.qweight.data_ptr(),
                                          tiles.data_ptr(), w.qzeros.data_ptr(), w.scales.data_ptr(), w.K, w.N,
                                          w.group_size, epilogue, _lib.ptr(residual), out.data_ptr(),
                                          _lib.ptr(out_up), _lib.ptr(next_norm), _lib.ptr(xg_out), _lib.ptr(ss_out),
                                          _lib.stream_handle(x2.device))
    _lib.check(rc, f"t2i_w4a16_linear_tiles_chain ({name})")


def linear_residual_next_norm(x: torch.Tensor, w: W4A16Weight, residual: torch.Tensor, out: torch.Tensor,
                              next_norm: torch.Tensor, xg_out: torch.Tensor, ss_out: torch.Tensor) -> torch.Tensor:
    """``out = bf16(bf16(x @ W^T) + residual)`` (``linear`` with a residual) that also
    writes the next RMSNorm's input: ``xg_out = bf16(out * next_norm)`` and ``ss_out``
    fp32 ``[M, N/16]``, the sums of ``out**2`` over each 16-column block."""
    _check_weight(w)
    for n_, t in (("x", x), ("residual", residual), ("out", out), ("next_norm", next_norm), ("xg_out", xg_out)):
        _check_dev(n_, t, BF16)
    _check_dev("ss_out", ss_out, torch.float32)
    m = x.shape[0]
    if x.shape != (m, w.K) or out.numel() != m * w.N or residual.numel() != m * w.N or xg_out.numel() != m * w.N:
        raise ValueError("x, residual, out and xg_out must be [M, K] / [M, N]")
    if next_norm.numel() != w.N or ss_out.numel() != m * (w.N // 16):
        raise ValueError("next_norm must hold N and ss_out M x N/16 values")
    _chain_call("producer", x, m, None, 0.0, w, _lib.T2I_TILES_STORE, residual, out, None, next_norm, xg_out, ss_out)
    return out


def _consumer_checks(xg, ss, w):
    _check_weight(w)
    _check_dev("xg", xg, BF16)
    _check_dev("ss", ss, torch.float32)
    m = xg.shape[0]
    if xg.dim() != 2 or xg.shape[1] != w.K or ss.numel() != m * (w.K // 16):
        raise ValueError("xg must be [M, K] and ss hold M x K/16 sums")
    return m


def prenormed_linear(xg: torch.Tensor, ss: torch.Tensor, eps: float, w: W4A16Weight,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """``rmsnorm_linear`` of the rows a ``linear_residual_next_norm`` call produced:
    ``xg`` is its ``xg_out`` (the rows times the norm weight) and ``ss`` its ``ss_out``."""
    m = _consumer_checks(xg, ss, w)
    if out is None:
        out = torch.empty(m, w.N, dtype=BF16, device=xg.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * w.N:
        raise ValueError(f"out must hold {m}x{w.N} elements")
    _chain_call("consumer", xg, m, ss, eps, w, _lib.T2I_TILES_STORE, None, out, None, None, None, None)
    return out


def prenormed_gate_up(xg: torch.Tensor, ss: torch.Tensor, eps: float, w_pair: W4A16Weight, swiglu: bool = True,
                      out: torch.Tensor | None = None, out_up: torch.Tensor | None = None):
    """``rmsnorm_gate_up`` of the rows a ``linear_residual_next_norm`` call produced."""
    m = _consumer_checks(xg, ss, w_pair)
    inter = w_pair.N // 2
    if out is None:
        out = torch.empty(m, inter, dtype=BF16, device=xg.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * inter:
        raise ValueError(f"out must hold {m}x{inter} elements")
    if not swiglu:
        if out_up is None:
            out_up = torch.empty(m, inter, dtype=BF16, device=xg.device)
        _check_dev("out_up", out_up, BF16)
    _chain_call("paired consumer", xg, m, ss, eps, w_pair, _lib.T2I_TILES_SWIGLU if swiglu else _lib.T2I_TILES_PAIRED,
                None, out, out_up, None, None, None)
    return out if swiglu else (out, out_up)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None,
            tokens: torch.Tensor | None = None, x_out: torch.Tensor | None = None,
            argmax_keys: torch.Tensor | None = None, out_sums: torch.Tensor | None = None) -> torch.Tensor:
    """Weighted RMSNorm of the rows of ``x`` (bf16 rounding as the reference's bf16 path).

    With ``tokens`` (int32 ``[M]``), ``x`` is an embedding table ``[V, H]`` and
    the gathered rows are also written to ``x_out``.  ``out_sums`` (fp32
    ``[H/128, M]``, not with ``argmax_keys``): each output row's sums over its
    128-wide groups, for a prompt GEMM that takes the output as ``x``.
    """
    _check_dev("x", x, BF16)
    _check_dev("weight", weight, BF16)
    h = x.shape[-1]
    if weight.numel() != h:
        raise ValueError("weight length must equal the row length")
    if tokens is not None:
        _check_dev("tokens", tokens, torch.int32)
        m = tokens.numel()
        if x.dim() != 2:
            raise ValueError("with tokens, x must be a [V, H] table")
        if x_out is None:
            raise ValueError("x_out is required with tokens")
    else:
        m = x.numel() // h
    if x_out is not None:
        _check_dev("x_out", x_out, BF16)
        if x_out.numel() != m * h:
            raise ValueError(f"x_out must hold {m}x{h} elements")
    if out is None:
        out = torch.empty(m, h, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != m * h:
        raise ValueError(f"out must hold {m}x{h} elements")
    if argmax_keys is not None:
        _check_dev("argmax_keys", argmax_keys, torch.int64)
        if argmax_keys.numel() < m:
            raise ValueError(f"argmax_keys must hold at least {m} entries")
    lib = _lib.load()
    if out_sums is not None:
        if argmax_keys is not None:
            raise ValueError("out_sums and argmax_keys are not taken together")
        _check_sums("out_sums", out_sums, m, h // 128)
        rc = lib.t2i_rmsnorm_sums(x.data_ptr(), _lib.ptr(tokens), x.shape[0] if tokens is not None else 0, m, h,
                                  weight.data_ptr(), float(eps), _lib.ptr(x_out), out.data_ptr(),
                                  out_sums.data_ptr(), _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_rmsnorm_sums")
        return out
    rc = lib.t2i_rmsnorm(x.data_ptr(), _lib.ptr(tokens), x.shape[0] if tokens is not None else 0, m, h,
                         weight.data_ptr(), float(eps), _lib.ptr(x_out),
                         out.data_ptr(), _lib.ptr(argmax_keys), _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_rmsnorm")
    return out


def decode_attention(qkv: torch.Tensor, positions: torch.Tensor, n_heads: int, n_kv_heads: int,
                     q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float, rope: torch.Tensor,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, rope_style: int = ROPE_HALVES,
                     out: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """q/k-norm + RoPE + KV write + GQA attention of one token per sequence.

    ``qkv`` bf16 ``[B, (Hq + 2 Hkv) * D]``, caches bf16 ``[B, Hkv, ctx_cap, D]``,
    ``rope`` bf16 ``[ctx_cap, D]`` (cos even / sin odd), ``positions`` int32 ``[B]``.
    Returns the context ``[B, Hq * D]`` (bf16).
    """
    _check_dev("qkv", qkv, BF16)
    _check_dev("positions", positions, torch.int32)
    for n, t in (("q_norm", q_norm), ("k_norm", k_norm), ("rope", rope), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_dev(n, t, BF16)
    b = positions.numel()
    d = q_norm.numel()
    if k_norm.numel() != d:
        raise ValueError("q_norm and k_norm must both hold head_dim values")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must be [B, Hkv, ctx_cap, D] of equal shape")
    if tuple(k_cache.shape[:2]) != (b, n_kv_heads) or k_cache.shape[3] != d:
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match B={b}, Hkv={n_kv_heads}, D={d}")
    ctx_cap = k_cache.shape[2]
    if rope.shape[0] < ctx_cap or rope.shape[1] != d:
        raise ValueError("rope table must be [>= ctx_cap, D]")
    if qkv.numel() != b * (n_heads + 2 * n_kv_heads) * d:
        raise ValueError("qkv must be [B, (Hq + 2 Hkv) * D]")
    if out is None:
        out = torch.empty(b, n_heads * d, dtype=BF16, device=qkv.device)
    _check_dev("out", out, BF16)
    if out.numel() != b * n_heads * d:
        raise ValueError(f"out must hold {b}x{n_heads * d} elements")
    lib = _lib.load()
    nbytes = lib.t2i_decode_attention_workspace_bytes(b, n_heads, n_kv_heads, ctx_cap)
    ws = (workspace or DEFAULT_WORKSPACE).get(("attn", b, n_kv_heads, ctx_cap), nbytes, qkv.device)
    rc = lib.t2i_decode_attention(qkv.data_ptr(), positions.data_ptr(), b, n_heads, n_kv_heads, d,
                                  q_norm.data_ptr(), k_norm.data_ptr(), float(eps), rope.data_ptr(), int(rope_style),
                                  k_cache.data_ptr(), v_cache.data_ptr(), ctx_cap, out.data_ptr(),
                                  _lib.ptr(ws), nbytes, _lib.stream_handle(qkv.device))
    _lib.check(rc, "t2i_decode_attention")
    return out


def decode_attention_prepared(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                              n_heads: int, n_kv_heads: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              out: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """KV write + GQA attention of one token per sequence whose q and k are
    normalised and rotated already (``rmsnorm_rope``): ``q`` bf16 ``[B, Hq * D]``,
    ``k`` / ``v`` bf16 ``[B, Hkv * D]``, caches ``[B, Hkv, ctx_cap, D]``.  Writes
    k and v at ``positions`` and returns the context ``[B, Hq * D]``."""
    for n, t in (("q", q), ("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_dev(n, t, BF16)
    _check_dev("positions", positions, torch.int32)
    b = positions.numel()
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must be [B, Hkv, ctx_cap, D] of equal shape")
    d = k_cache.shape[3]
    if tuple(k_cache.shape[:2]) != (b, n_kv_heads):
        raise ValueError(f"cache shape {tuple(k_cache.shape)} does not match B={b}, Hkv={n_kv_heads}")
    if q.numel() != b * n_heads * d or k.numel() != b * n_kv_heads * d or v.numel() != b * n_kv_heads * d:
        raise ValueError("q must be [B, Hq * D] and k, v [B, Hkv * D]")
    ctx_cap = k_cache.shape[2]
    if out is None:
        out = torch.empty(b, n_heads * d, dtype=BF16, device=q.device)
    _check_dev("out", out, BF16)
    if out.numel() != b * n_heads * d:
        raise ValueError(f"out must hold {b}x{n_heads * d} elements")
    lib = _lib.load()
    nbytes = lib.t2i_decode_attention_workspace_bytes(b, n_heads, n_kv_heads, ctx_cap)
    ws = (workspace or DEFAULT_WORKSPACE).get(("attn", b, n_kv_heads, ctx_cap), nbytes, q.device)
    rc = lib.t2i_decode_attention_prepared(q.data_ptr(), k.data_ptr(), v.data_ptr(), positions.data_ptr(), b,
                                           n_heads, n_kv_heads, d, k_cache.data_ptr(), v_cache.data_ptr(), ctx_cap,
                                           out.data_ptr(), _lib.ptr(ws), nbytes, _lib.stream_handle(q.device))
    _lib.check(rc, "t2i_decode_attention_prepared")
    return out


def rmsnorm_rope(x: torch.Tensor, weight: torch.Tensor, angles: torch.Tensor, eps: float,
                 rope_style: int = ROPE_HALVES, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-row weighted RMSNorm then RoPE: ``x`` bf16 ``[rows, cols]``, ``weight``
    ``[cols]``, ``angles`` ``[angle_rows, cols]`` (cos even / sin odd); row r takes
    angle row ``r // (rows // angle_rows)``.  ``out`` may be ``x``."""
    for n, t in (("x", x), ("weight", weight), ("angles", angles)):
        _check_dev(n, t, BF16)
    cols = weight.numel()
    if x.numel() % cols or angles.numel() % cols:
        raise ValueError("x and angles must hold whole rows of len(weight) values")
    rows, angle_rows = x.numel() // cols, angles.numel() // cols
    if out is None:
        out = torch.empty_like(x)
    _check_dev("out", out, BF16)
    if out.numel() != x.numel():
        raise ValueError("out must match x")
    lib = _lib.load()
    rc = lib.t2i_rmsnorm_rope(x.data_ptr(), rows, cols, weight.data_ptr(), angles.data_ptr(), angle_rows,
                              float(eps), int(rope_style), out.data_ptr(), _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_rmsnorm_rope")
    return out


def silu_mul(left: torch.Tensor, right: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``bf16(bf16(silu(left)) * right)`` elementwise (bf16 tensors of equal size)."""
    _check_dev("left", left, BF16)
    _check_dev("right", right, BF16)
    if left.numel() != right.numel():
        raise ValueError("left and right must hold the same number of values")
    if out is None:
        out = torch.empty_like(left)
    _check_dev("out", out, BF16)
    if out.numel() != left.numel():
        raise ValueError("out must match left")
    lib = _lib.load()
    rc = lib.t2i_silu_mul(left.data_ptr(), right.data_ptr(), left.numel(), out.data_ptr(),
                          _lib.stream_handle(left.device))
    _lib.check(rc, "t2i_silu_mul")
    return out


def residual_add_rmsnorm(x: torch.Tensor, update: torch.Tensor, weight: torch.Tensor, eps: float,
                         x_out: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """``x_out = bf16(x + update)`` and ``out = rmsnorm(x_out) * weight`` over rows of
    ``len(weight)`` (``x_out`` may be ``x``).  Returns ``(x_out, out)``."""
    for n, t in (("x", x), ("update", update), ("weight", weight)):
        _check_dev(n, t, BF16)
    h = weight.numel()
    if x.numel() % h or update.numel() != x.numel():
        raise ValueError("x and update must be whole rows of len(weight) values, of equal size")
    m = x.numel() // h
    x_out = torch.empty_like(x) if x_out is None else x_out
    out = torch.empty_like(x) if out is None else out
    for n, t in (("x_out", x_out), ("out", out)):
        _check_dev(n, t, BF16)
        if t.numel() != x.numel():
            raise ValueError(f"{n} must match x")
    lib = _lib.load()
    rc = lib.t2i_residual_add_rmsnorm(x.data_ptr(), update.data_ptr(), m, h, weight.data_ptr(), float(eps),
                                      x_out.data_ptr(), out.data_ptr(), _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_residual_add_rmsnorm")
    return x_out, out


def qkv_attention(x: torch.Tensor, norm_weight: torch.Tensor | None, eps: float, w_qkv: W4A16Weight,
                  positions: torch.Tensor, n_heads: int, n_kv_heads: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                  rope: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, rope_style: int = ROPE_HALVES,
                  out: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """The decode layer's front in one cooperative launch: RMSNorm (``norm_weight``,
    or none when ``x`` is already normalised) + the fused q|k|v projection, then
    ``decode_attention`` on those rows.  ``x`` bf16 ``[B, hidden]`` (B <= 16); returns
    the context ``[B, Hq * D]``.  The launch takes one workgroup per CU: it must not
    run concurrently with other GPU work."""
    _check_weight(w_qkv)
    _check_dev("x", x, BF16)
    _check_dev("positions", positions, torch.int32)
    for n, t in (("q_norm", q_norm), ("k_norm", k_norm), ("rope", rope), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_dev(n, t, BF16)
    if norm_weight is not None:
        _check_dev("norm_weight", norm_weight, BF16)
        if norm_weight.numel() != w_qkv.K:
            raise ValueError("norm_weight must hold K values")
    b = positions.numel()
    d = q_norm.numel()
    if k_norm.numel() != d:
        raise ValueError("q_norm and k_norm must both hold head_dim values")
    if x.numel() != b * w_qkv.K:
        raise ValueError(f"x must be [B, {w_qkv.K}] with B = {b}")
    if w_qkv.N != (n_heads + 2 * n_kv_heads) * d:
        raise ValueError("the qkv weight must have (Hq + 2 Hkv) * D columns")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or tuple(k_cache.shape[:2]) != (b, n_kv_heads) \
            or k_cache.shape[3] != d:
        raise ValueError("caches must be [B, Hkv, ctx_cap, D]")
    ctx_cap = k_cache.shape[2]
    if rope.shape[0] < ctx_cap or rope.shape[1] != d:
        raise ValueError("rope table must be [>= ctx_cap, D]")
    if out is None:
        out = torch.empty(b, n_heads * d, dtype=BF16, device=x.device)
    _check_dev("out", out, BF16)
    if out.numel() != b * n_heads * d:
        raise ValueError(f"out must hold {b}x{n_heads * d} elements")
    lib = _lib.load()
    nbytes = lib.t2i_qkv_attention_workspace_bytes(b, n_heads, n_kv_heads)
    if nbytes == 0:
        raise ValueError(f"unsupported shape for the fused launch: B={b}, Hq={n_heads}, Hkv={n_kv_heads}")
    ws = (workspace or DEFAULT_WORKSPACE).get(("qkv_attn", b, n_heads, n_kv_heads), nbytes, x.device)
    rc = lib.t2i_qkv_attention(x.data_ptr(), b, _lib.ptr(norm_weight), float(eps), w_qkv.qweight.data_ptr(),
                               w_qkv.qzeros.data_ptr(), w_qkv.scales.data_ptr(), w_qkv.K, w_qkv.group_size,
                               positions.data_ptr(), n_heads, n_kv_heads, d, q_norm.data_ptr(), k_norm.data_ptr(),
                               rope.data_ptr(), int(rope_style), k_cache.data_ptr(), v_cache.data_ptr(), ctx_cap,
                               out.data_ptr(), ws.data_ptr(), nbytes, _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_qkv_attention")
    return out


def qkv_attention_errors(b: int, n_heads: int, n_kv_heads: int, device, workspace: Workspace | None = None) -> int:
    """The error word of the fused launch's workspace (non-zero: a wait timed out).
    Synchronises with the device."""
    lib = _lib.load()
    off = lib.t2i_qkv_attention_error_offset(b, n_heads, n_kv_heads)
    nbytes = lib.t2i_qkv_attention_workspace_bytes(b, n_heads, n_kv_heads)
    ws = (workspace or DEFAULT_WORKSPACE).get(("qkv_attn", b, n_heads, n_kv_heads), nbytes, device)
    return int(ws[off:off + 4].view(torch.int32).item())


def clear_qkv_attention_errors(b: int, n_heads: int, n_kv_heads: int, device,
                               workspace: Workspace | None = None) -> None:
    """Zero the fused launch's error word (a fill kernel on torch's current
    stream), so that later launches wait normally again."""
    lib = _lib.load()
    off = lib.t2i_qkv_attention_error_offset(b, n_heads, n_kv_heads)
    nbytes = lib.t2i_qkv_attention_workspace_bytes(b, n_heads, n_kv_heads)
    ws = (workspace or DEFAULT_WORKSPACE).get(("qkv_attn", b, n_heads, n_kv_heads), nbytes, device)
    ws[off:off + 4].zero_()


class DecodeLayerTable:
    """The per-layer weights and caches of ``decode_step``: a device array of
    ``t2i_decode_layer`` entries (18 pointers a layer, in the header's field
    order), checked once here and kept alive with the tensors it points into.

    ``layers``: one dict per layer with W4A16Weight ``qkv`` (q|k|v columns),
    ``o``, ``gate_up`` (``interleave_gate_up`` layout), ``down``; bf16 ``ln1``,
    ``ln2`` [hidden], ``q_norm``, ``k_norm`` [D]; bf16 caches ``k_cache``,
    ``v_cache`` [B, Hkv, ctx_cap, D].
    """

    FIELDS = ("qkv", "o", "gate_up", "down")

    def __init__(self, layers: list, n_heads: int, n_kv_heads: int, device):
        if not layers:
            raise ValueError("at least one layer")
        d = layers[0]["q_norm"].numel()
        kc0 = layers[0]["k_cache"]
        if kc0.dim() != 4:
            raise ValueError("caches must be [B, Hkv, ctx_cap, D]")
        self.batch, self.ctx_cap = kc0.shape[0], kc0.shape[2]
        self.hidden = layers[0]["ln1"].numel()
        self.intermediate = layers[0]["gate_up"].N // 2
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, d
        self.n_layers = len(layers)
        h, i = self.hidden, self.intermediate
        shapes = {"qkv": (h, (n_heads + 2 * n_kv_heads) * d), "o": (n_heads * d, h), "gate_up": (h, 2 * i),
                  "down": (i, h)}
        rows = []
        for li, lay in enumerate(layers):
            row = []
            for f in self.FIELDS:
                w = lay[f]
                _check_weight(w)
                if (w.K, w.N) != shapes[f] or w.group_size != GROUP_SIZE:
                    raise ValueError(f"layer {li}: {f} must be K x N = {shapes[f]}, group {GROUP_SIZE}")
                row += [w.qweight.data_ptr(), w.qzeros.data_ptr(), w.scales.data_ptr()]
            for f, n in (("ln1", h), ("ln2", h), ("q_norm", d), ("k_norm", d)):
                _check_dev(f, lay[f], BF16)
                if lay[f].numel() != n:
                    raise ValueError(f"layer {li}: {f} must hold {n} values")
                row.append(lay[f].data_ptr())
            for f in ("k_cache", "v_cache"):
                c = lay[f]
                _check_dev(f, c, BF16)
                if tuple(c.shape) != (self.batch, n_kv_heads, self.ctx_cap, d):
                    raise ValueError(f"layer {li}: {f} must be [{self.batch}, {n_kv_heads}, {self.ctx_cap}, {d}]")
                row.append(c.data_ptr())
            rows.append(row)
        self._keep = layers
        self.table = torch.tensor(rows, dtype=torch.int64).to(device)

    def workspace_bytes(self) -> int:
        """0 when the library has no one-launch plan for these shapes."""
        return _lib.load().t2i_decode_step_workspace_bytes(self.batch, self.n_layers, self.hidden, self.intermediate,
                                                           self.n_heads, self.n_kv_heads)

    def _key(self):
        return ("decode_step", self.batch, self.n_layers, self.hidden, self.intermediate, self.n_heads,
                self.n_kv_heads)


def decode_step(table: DecodeLayerTable, xn0: torch.Tensor, x: torch.Tensor, positions: torch.Tensor,
                eps: float, rope: torch.Tensor, rope_style: int = ROPE_HALVES,
                workspace: Workspace | None = None) -> torch.Tensor:
    """Every decoder layer of one decode step in one cooperative launch
    (``t2i_decode_step``).  ``xn0`` bf16 ``[B, hidden]``: layer 0's normalised
    input; ``x``: the residual stream, the embedding rows in and the last
    layer's output out (updated in place and returned).  The launch takes one
    workgroup per CU: it must not run concurrently with other GPU work."""
    if not isinstance(table, DecodeLayerTable):
        raise ValueError("table must be a DecodeLayerTable")
    b, h = table.batch, table.hidden
    for n, t in (("xn0", xn0), ("x", x), ("rope", rope)):
        _check_dev(n, t, BF16)
    _check_dev("positions", positions, torch.int32)
    if xn0.numel() != b * h or x.numel() != b * h:
        raise ValueError(f"xn0 and x must be [{b}, {h}]")
    if positions.numel() != b:
        raise ValueError(f"positions must hold {b} values")
    if rope.dim() != 2 or rope.shape[0] < table.ctx_cap or rope.shape[1] != table.head_dim:
        raise ValueError("rope table must be [>= ctx_cap, D]")
    nbytes = table.workspace_bytes()
    if nbytes == 0:
        raise ValueError("no one-launch decode-step plan for these shapes")
    ws = (workspace or DEFAULT_WORKSPACE).get(table._key(), nbytes, x.device)
    lib = _lib.load()
    rc = lib.t2i_decode_step(table.table.data_ptr(), table.n_layers, xn0.data_ptr(), x.data_ptr(), b, h,
                             table.intermediate, table.n_heads, table.n_kv_heads, table.head_dim, GROUP_SIZE,
                             positions.data_ptr(), rope.data_ptr(), int(rope_style), table.ctx_cap, float(eps),
                             ws.data_ptr(), nbytes, _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_decode_step")
    return x


def _step_region(table: DecodeLayerTable, which: int, device, workspace: Workspace | None):
    lib = _lib.load()
    args = (table.batch, table.n_layers, table.hidden, table.intermediate, table.n_heads, table.n_kv_heads)
    ws = (workspace or DEFAULT_WORKSPACE).get(table._key(), lib.t2i_decode_step_workspace_bytes(*args), device)
    return ws, lib.t2i_decode_step_offset(*args, which)


def decode_step_errors(table: DecodeLayerTable, device, workspace: Workspace | None = None) -> int:
    """The error word of the one-launch step's workspace (non-zero: a wait timed
    out).  Synchronises with the device."""
    ws, off = _step_region(table, 4, device, workspace)
    return int(ws[off:off + 4].view(torch.int32).item())


def clear_decode_step_errors(table: DecodeLayerTable, device, workspace: Workspace | None = None) -> None:
    """Zero the one-launch step's error word (a fill kernel on torch's current
    stream), so that later launches wait normally again."""
    ws, off = _step_region(table, 4, device, workspace)
    ws[off:off + 4].zero_()


def decode_step_intermediates(table: DecodeLayerTable, device, workspace: Workspace | None = None) -> dict:
    """Copies of the last one-launch step's per-layer activations from its
    workspace's tagged words (for checks): ``ctx`` [L, B, Hq*D], ``xmid``
    [L, B, hidden] (after attention), ``h`` [L, B, intermediate] (SwiGLU), ``x``
    [L-1, B, hidden] (between layers), ``qkv`` [B, (Hq+2Hkv)*D] (the last layer's
    projection)."""
    b, L, h, i, d = table.batch, table.n_layers, table.hidden, table.intermediate, table.head_dim
    hq, hkv = table.n_heads, table.n_kv_heads
    def low16(words):
        v = words.to(torch.int64) & 0xFFFF
        return torch.where(v >= 32768, v - 65536, v).to(torch.int16).view(BF16)

    views = {}
    for which, name, shape in ((0, "ctx", (L, b, hq * d)), (1, "xmid", (L, b, h)), (2, "h", (L, b, i)),
                               (3, "x", (max(L - 1, 1), b, h))):
        ws, off = _step_region(table, which, device, workspace)
        n = shape[0] * shape[1] * shape[2]
        views[name] = low16(ws[off:off + 4 * n].view(torch.int32)).view(shape)
    nq = (hq + 2 * hkv) * d
    ws, _ = _step_region(table, 0, device, workspace)
    views["qkv"] = low16(ws[:b * nq * 8].view(torch.int64)).view(b, nq)
    return views


def prefill_qk_rope_kv(qkv: torch.Tensor, batch: int, p0: int, n_heads: int, n_kv_heads: int,
                       q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float, rope: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, rope_style: int = ROPE_HALVES,
                       q_out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + RoPE of every prompt row and the KV-cache write of positions p0..p0+T-1.

    ``qkv`` bf16 ``[B * T, (Hq + 2 Hkv) * D]`` (row ``b * T + t``); returns q
    bf16 ``[B, Hq, T, D]``.
    """
    _check_dev("qkv", qkv, BF16)
    for n, t in (("q_norm", q_norm), ("k_norm", k_norm), ("rope", rope), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_dev(n, t, BF16)
    d = q_norm.numel()
    if k_norm.numel() != d:
        raise ValueError("q_norm and k_norm must both hold head_dim values")
    if batch < 1:
        raise ValueError("batch must be positive")
    rows = qkv.numel() // ((n_heads + 2 * n_kv_heads) * d)
    if rows % batch or rows * (n_heads + 2 * n_kv_heads) * d != qkv.numel():
        raise ValueError("qkv must be [B * T, (Hq + 2 Hkv) * D]")
    t = rows // batch
    if (k_cache.dim() != 4 or k_cache.shape != v_cache.shape or tuple(k_cache.shape[:2]) != (batch, n_kv_heads)
            or k_cache.shape[3] != d):
        raise ValueError("caches must be [B, Hkv, ctx_cap, D]")
    ctx_cap = k_cache.shape[2]
    if rope.dim() != 2 or rope.shape[0] < p0 + t or rope.shape[1] != d:
        raise ValueError("rope must be [>= p0 + T positions, D]")
    if q_out is None:
        q_out = torch.empty(batch, n_heads, t, d, dtype=BF16, device=qkv.device)
    _check_dev("q_out", q_out, BF16)
    if q_out.numel() != batch * n_heads * t * d:
        raise ValueError("q_out must be [B, Hq, T, D]")
    lib = _lib.load()
    rc = lib.t2i_prefill_qk_rope_kv(qkv.data_ptr(), batch, t, p0, n_heads, n_kv_heads, d, q_norm.data_ptr(),
                                    k_norm.data_ptr(), float(eps), rope.data_ptr(), int(rope_style),
                                    q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), ctx_cap,
                                    _lib.stream_handle(qkv.device))
    _lib.check(rc, "t2i_prefill_qk_rope_kv")
    return q_out


def prefill_qkv_rope_kv(x: torch.Tensor, w_qkv: W4A16Weight, batch: int, p0: int, n_heads: int, n_kv_heads: int,
                        q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float, rope: torch.Tensor,
                        k_cache: torch.Tensor, v_cache: torch.Tensor, rope_style: int = ROPE_HALVES,
                        q_out: torch.Tensor | None = None, x_sums: torch.Tensor | None = None) -> torch.Tensor:
    """``prefill_qk_rope_kv(linear(x, w_qkv), ...)`` in one launch, with the same bits:
    the prompt GEMM's epilogue normalises and rotates each q/k head and writes q
    and the caches, and the projection is never stored.  ``x`` bf16 ``[B * T, K]``
    with ``B * T >= 512`` (the prompt GEMM's rows); returns q bf16 ``[B, Hq, T, D]``.
    ``x_sums`` as ``linear`` (``sum_parts=1``)."""
    _check_dev("x", x, BF16)
    _check_weight(w_qkv)
    for n, t in (("q_norm", q_norm), ("k_norm", k_norm), ("rope", rope), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check_dev(n, t, BF16)
    d = q_norm.numel()
    if k_norm.numel() != d:
        raise ValueError("q_norm and k_norm must both hold head_dim values")
    if batch < 1 or x.dim() != 2 or x.shape[0] % batch:
        raise ValueError("x must be [B * T, K] with B = batch")
    if x.shape[1] != w_qkv.K or w_qkv.N != (n_heads + 2 * n_kv_heads) * d:
        raise ValueError("w_qkv must be [K = x.shape[1], (Hq + 2 Hkv) * D]")
    t = x.shape[0] // batch
    if (k_cache.dim() != 4 or k_cache.shape != v_cache.shape or tuple(k_cache.shape[:2]) != (batch, n_kv_heads)
            or k_cache.shape[3] != d):
        raise ValueError("caches must be [B, Hkv, ctx_cap, D]")
    ctx_cap = k_cache.shape[2]
    if rope.dim() != 2 or rope.shape[0] < p0 + t or rope.shape[1] != d:
        raise ValueError("rope must be [>= p0 + T positions, D]")
    if q_out is None:
        q_out = torch.empty(batch, n_heads, t, d, dtype=BF16, device=x.device)
    _check_dev("q_out", q_out, BF16)
    if q_out.numel() != batch * n_heads * t * d:
        raise ValueError("q_out must be [B, Hq, T, D]")
    lib = _lib.load()
    if x_sums is not None:
        _check_sums("x_sums", x_sums, x.shape[0], w_qkv.K // w_qkv.group_size)
        rc = lib.t2i_prefill_qkv_rope_kv_sums(x.data_ptr(), x_sums.data_ptr(), batch, t, p0,
                                              w_qkv.qweight.data_ptr(), w_qkv.qzeros.data_ptr(),
                                              w_qkv.scales.data_ptr(), w_qkv.K, w_qkv.group_size, n_heads,
                                              n_kv_heads, d, q_norm.data_ptr(), k_norm.data_ptr(), float(eps),
                                              rope.data_ptr(), int(rope_style), q_out.data_ptr(),
                                              k_cache.data_ptr(), v_cache.data_ptr(), ctx_cap,
                                              _lib.stream_handle(x.device))
        _lib.check(rc, "t2i_prefill_qkv_rope_kv_sums")
        return q_out
    rc = lib.t2i_prefill_qkv_rope_kv(x.data_ptr(), batch, t, p0, w_qkv.qweight.data_ptr(), w_qkv.qzeros.data_ptr(),
                                     w_qkv.scales.data_ptr(), w_qkv.K, w_qkv.group_size, n_heads, n_kv_heads, d,
                                     q_norm.data_ptr(), k_norm.data_ptr(), float(eps), rope.data_ptr(),
                                     int(rope_style), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                     ctx_cap, _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_prefill_qkv_rope_kv")
    return q_out


def prefill_attention(q: torch.Tensor, p0: int, n_kv_heads: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      out: torch.Tensor | None = None, out_sums: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA attention of prompt rows ``q [B, Hq, T, D]`` (positions p0..p0+T-1)
    over cache slots ``0..p0+t``; returns bf16 ``[B * T, Hq * D]``.  ``out_sums``
    (fp32 ``[Hq, B * T]``) receives each head's sum of its bf16 context values,
    the o_proj's ``x_sums`` when ``D = 128``."""
    _check_dev("q", q, BF16)
    _check_dev("k_cache", k_cache, BF16)
    _check_dev("v_cache", v_cache, BF16)
    if q.dim() != 4:
        raise ValueError("q must be [B, Hq, T, D]")
    b, hq, t, d = q.shape
    if (k_cache.dim() != 4 or k_cache.shape != v_cache.shape or tuple(k_cache.shape[:2]) != (b, n_kv_heads)
            or k_cache.shape[3] != d):
        raise ValueError("caches must be [B, Hkv, ctx_cap, D]")
    if out is None:
        out = torch.empty(b * t, hq * d, dtype=BF16, device=q.device)
    _check_dev("out", out, BF16)
    if out.numel() != b * t * hq * d:
        raise ValueError("out must be [B * T, Hq * D]")
    lib = _lib.load()
    if out_sums is not None:
        _check_sums("out_sums", out_sums, b * t, hq)
        rc = lib.t2i_prefill_attention_sums(q.data_ptr(), b, t, p0, hq, n_kv_heads, d, k_cache.data_ptr(),
                                            v_cache.data_ptr(), k_cache.shape[2], out.data_ptr(),
                                            out_sums.data_ptr(), _lib.stream_handle(q.device))
        _lib.check(rc, "t2i_prefill_attention_sums")
        return out
    rc = lib.t2i_prefill_attention(q.data_ptr(), b, t, p0, hq, n_kv_heads, d, k_cache.data_ptr(),
                                   v_cache.data_ptr(), k_cache.shape[2], out.data_ptr(),
                                   _lib.stream_handle(q.device))
    _lib.check(rc, "t2i_prefill_attention")
    return out


def lm_head_argmax(h: torch.Tensor, embed: torch.Tensor, keys: torch.Tensor,
                   logits: torch.Tensor | None = None) -> torch.Tensor:
    """Tied bf16 lm_head + greedy argmax into ``keys`` (int64 ``[M]``, zeroed beforehand)."""
    _check_dev("h", h, BF16)
    _check_dev("embed", embed, BF16)
    _check_dev("keys", keys, torch.int64)
    if h.dim() != 2 or embed.dim() != 2:
        raise ValueError("h must be [M, K] and embed [V, K]")
    m, k = h.shape
    v = embed.shape[0]
    if embed.shape[1] != k:
        raise ValueError("embed must be [V, K] with K = h.shape[1]")
    if keys.numel() < m:
        raise ValueError(f"keys must hold at least {m} entries")
    if logits is not None:
        _check_dev("logits", logits, torch.float32)
        if logits.numel() != m * v:
            raise ValueError("logits must be [M, V]")
    lib = _lib.load()
    rc = lib.t2i_lm_head_argmax(h.data_ptr(), m, embed.data_ptr(), v, k, _lib.ptr(logits), keys.data_ptr(),
                                _lib.stream_handle(h.device))
    _lib.check(rc, "t2i_lm_head_argmax")
    return keys


def rmsnorm_lm_head_argmax(x: torch.Tensor, weight: torch.Tensor, eps: float, embed: torch.Tensor,
                           keys: torch.Tensor, logits: torch.Tensor | None = None) -> torch.Tensor:
    """``lm_head_argmax(rmsnorm(x, weight, eps), embed, keys, logits)`` in one launch, with
    the same bits (``keys`` zeroed beforehand; the hidden size a power of two)."""
    _check_dev("x", x, BF16)
    _check_dev("weight", weight, BF16)
    _check_dev("embed", embed, BF16)
    _check_dev("keys", keys, torch.int64)
    if x.dim() != 2 or embed.dim() != 2:
        raise ValueError("x must be [M, K] and embed [V, K]")
    m, k = x.shape
    v = embed.shape[0]
    if embed.shape[1] != k or weight.numel() != k:
        raise ValueError("embed must be [V, K] and weight [K] with K = x.shape[1]")
    if keys.numel() < m:
        raise ValueError(f"keys must hold at least {m} entries")
    if logits is not None:
        _check_dev("logits", logits, torch.float32)
        if logits.numel() != m * v:
            raise ValueError("logits must be [M, V]")
    lib = _lib.load()
    rc = lib.t2i_rmsnorm_lm_head_argmax(x.data_ptr(), m, weight.data_ptr(), float(eps), embed.data_ptr(), v, k,
                                        _lib.ptr(logits), keys.data_ptr(), _lib.stream_handle(x.device))
    _lib.check(rc, "t2i_rmsnorm_lm_head_argmax")
    return keys


def keys_to_tokens(keys: torch.Tensor) -> torch.Tensor:
    """Decode argmax keys (``ordered << 32 | (0xFFFFFFFF - index)``) into indices."""
    low = keys & 0xFFFFFFFF
    return (0xFFFFFFFF - low).to(torch.int64)


def greedy_advance(keys, tokens, positions, history, step):
    """Device-side greedy bookkeeping between captured decode steps (``history`` may
    be None: no token record)."""
    _check_dev("keys", keys, torch.int64)
    _check_dev("tokens", tokens, torch.int32)
    _check_dev("positions", positions, torch.int32)
    _check_dev("step", step, torch.int32)
    b = tokens.numel()
    if keys.numel() < b or positions.numel() != b or step.numel() < 1:
        raise ValueError("keys, tokens and positions must hold one entry per sequence; step one")
    if history is not None:
        _check_dev("history", history, torch.int32)
        if history.dim() != 2 or history.shape[0] != b:
            raise ValueError("history must be [B, hist_cap]")
    lib = _lib.load()
    rc = lib.t2i_greedy_advance(keys.data_ptr(), b, tokens.data_ptr(), positions.data_ptr(),
                                history.data_ptr() if history is not None else None,
                                history.shape[1] if history is not None else 0, step.data_ptr(),
                                _lib.stream_handle(tokens.device))
    _lib.check(rc, "t2i_greedy_advance")


def prompt_advance(prompt, tokens, positions):
    """Teacher-forced prompt bookkeeping (``prompt`` int32 ``[B, P]``)."""
    _check_dev("prompt", prompt, torch.int32)
    _check_dev("tokens", tokens, torch.int32)
    _check_dev("positions", positions, torch.int32)
    if prompt.dim() != 2 or tokens.numel() != prompt.shape[0] or positions.numel() != prompt.shape[0]:
        raise ValueError("prompt must be [B, P] with one token and position per sequence")
    lib = _lib.load()
    b, plen = prompt.shape
    rc = lib.t2i_prompt_advance(prompt.data_ptr(), b, plen, tokens.data_ptr(), positions.data_ptr(),
                                _lib.stream_handle(tokens.device))
    _lib.check(rc, "t2i_prompt_advance")


def stream_read(src, nbytes: int | None = None, offset: int = 0, loads_per_thread: int = 4, out=None):
    """Read ``nbytes`` of ``src`` from byte ``offset`` with the HBM read-ceiling
    kernel (``t2i_stream_read``) and return the per-wave XOR words (uint32 bit
    patterns in an int32 tensor).  ``offset`` and ``nbytes`` must be multiples of
    16; ``out`` may be a preallocated int32 tensor of at least the word count."""
    _check_dev("src", src)
    total = src.numel() * src.element_size()
    nbytes = total - offset if nbytes is None else nbytes
    if offset < 0 or nbytes <= 0 or offset % 16 or nbytes % 16 or offset + nbytes > total:
        raise ValueError(f"bytes [{offset}, {offset + nbytes}) must be 16-aligned and inside the {total}-byte source")
    lib = _lib.load()
    words = lib.t2i_stream_read_out_words(nbytes, loads_per_thread)
    if words <= 0:
        raise ValueError(f"loads_per_thread must be 1, 2, 4 or 8 (got {loads_per_thread})")
    if out is None:
        out = torch.empty(words, dtype=torch.int32, device=src.device)
    else:
        _check_dev("out", out, torch.int32)
        if out.numel() < words:
            raise ValueError(f"out holds {out.numel()} words, {words} needed")
    rc = lib.t2i_stream_read(src.data_ptr() + offset, nbytes, loads_per_thread, out.data_ptr(),
                             _lib.stream_handle(src.device))
    _lib.check(rc, "t2i_stream_read")
    return out[:words]
