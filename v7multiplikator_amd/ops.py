"""Torch-facing host API of the fused per-layer kernels.

Mirrors the reference's kernel entry points (src/v7_lib.h:113-128,269-281) for
batched device tensors.  Every function validates its tensors, binds the
library to torch's current stream and makes ONE launch through the C ABI of
libv7g.so; nothing runs on the CPU and there is no fallback: without the built
library the first call raises.

  fused_add_rmsnorm  <- v7s_fused_add_rmsnorm   (src/asm/add_rmsnorm_kernel.inc:15-129)
  rmsnorm            <- v7s_rmsnorm             (src/asm/rmsnorm_kernel.inc:12-75)
  rmsnorm_quantize   <- v7s_rmsnorm_quantize    (src/asm/rmsnorm_quantize_kernel.inc:62-218)
  add_rmsnorm_quantize <- v7s_add_inplace then v7s_rmsnorm_quantize, one pass (src/asm/forward_q8.inc:386-387)
  add_inplace        <- v7s_add_inplace         (src/asm/add_kernel.inc:26-49)
  rmsnorm_rope_heads <- v7s_rmsnorm_rope_heads  (src/asm/rmsnorm_rope_dispatch.inc:11-52)
  qk_rmsnorm_rope    <- v7s_qk_fork_heads, both sides in one launch (src/asm/qk_fork_kernel.inc:40-62)
  swiglu             <- .pq_ffn_silu            (src/asm/prefill_q8.inc:1159-1166)
  quantize_q8        <- v7d_quantize            (src/asm/utility_dispatch.inc:108-212)
  swiglu_q8          <- SwiGLU then v7d_quantize (src/asm/prefill_q8.inc:1154-1183)
  embedding_gather_q8 <- v7s_embedding_row      (src/asm/forward.inc:13-42)
  rope_tables        <- v7s_rope_init           (src/asm/fused_dispatch.inc:58-76; Llama 3 scaling
                                                  src/asm/fused_f32_kernel.inc:149-256)
  kv_pack_f16        <- v7s_kv_pack_f16         (src/asm/kv_f16c.inc:12-52)
  kv_pack_f16_kv     <- v7s_kv_pack_f16 for K then V (src/asm/forward_q8.inc:345-358), one launch
  rope_only_heads    <- v7s_rope_only_heads     (src/asm/rope_only_dispatch.inc:11-47)
  qkv_rope_stage     <- the per-token Q/K/V stage of the prefill, one launch (src/asm/prefill_q8.inc:848-883)
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

Q8_EMBED_GS = 64  # scale group of the Q8 embedding table (src/asm/forward.inc:14, GS=64)


# torch's current stream of a device as a raw handle: the query torch's own generated code makes (about 0.1 us
# per call, against about 2 us for torch.cuda.current_stream(), which builds a Stream object); the public call
# where this torch lacks it.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on `device`.  If the raw query rejects its argument (a torch
    that changed its signature), the public call takes over for the rest of the process."""
    global _raw_stream
    if _raw_stream is not None:
        try:
            return _raw_stream(device.index)
        except (TypeError, RuntimeError):
            _raw_stream = None
    return torch.cuda.current_stream(device).cuda_stream


def _bind(t: torch.Tensor) -> None:
    """Binds the calling thread's library stream to torch's current stream of t's device."""
    if not t.is_cuda:
        raise ValueError("v7g kernels take device tensors (cuda:N)")
    _lib.load().v7g_set_stream(current_stream_handle(t.device))


def _need(t: torch.Tensor, dtype, name: str, contiguous: bool = True) -> None:
    """Every tensor of a call lives on the current device, where the library launches."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a cuda device")
    cur = torch.cuda.current_device()
    if t.device.index != cur:
        raise ValueError(f"{name} is on {t.device} but the current device is cuda:{cur}; "
                         f"call under torch.cuda.device({t.device})")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def fused_add_rmsnorm(residual: torch.Tensor, add: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """residual += add (in place); returns out = rmsnorm(residual) * weight.  [rows, dim] f32."""
    for t, n in ((residual, "residual"), (add, "add"), (weight, "weight")):
        _need(t, torch.float32, n)
    dim = residual.shape[-1]
    rows = residual.numel() // dim if dim else 0
    if add.shape != residual.shape or weight.numel() != dim:
        raise ValueError("shape mismatch: add must match residual, weight must be [dim]")
    if out is None:
        out = torch.empty_like(residual)
    _need(out, torch.float32, "out")
    if out.shape != residual.shape:
        raise ValueError("out must match residual")
    _bind(residual)
    rc = _lib.load().v7g_fused_add_rmsnorm(out.data_ptr(), residual.data_ptr(), add.data_ptr(), weight.data_ptr(),
                                           rows, dim, float(eps))
    _lib.check(rc, "fused_add_rmsnorm")
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = rmsnorm(x) * weight per row of x [rows, dim] (dim % 32 == 0); out may be x."""
    _need(x, torch.float32, "x")
    _need(weight, torch.float32, "weight")
    dim = x.shape[-1]
    if weight.numel() != dim:
        raise ValueError("weight must be [dim]")
    if out is None:
        out = torch.empty_like(x)
    _need(out, torch.float32, "out")
    if out.shape != x.shape:
        raise ValueError("out must match x")
    _bind(x)
    rc = _lib.load().v7g_rmsnorm(out.data_ptr(), x.data_ptr(), weight.data_ptr(), x.numel() // dim if dim else 0, dim,
                                 float(eps))
    _lib.check(rc, "rmsnorm")
    return out


def rmsnorm_quantize(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, gs: int = 64,
                     out_q: torch.Tensor | None = None, out_s: torch.Tensor | None = None):
    """RMSNorm then Q8 per row of x [rows, dim]: returns (codes int8 like x, scales [rows, dim/gs])."""
    _need(x, torch.float32, "x")
    _need(weight, torch.float32, "weight")
    dim = x.shape[-1]
    if weight.numel() != dim:
        raise ValueError("weight must be [dim]")
    rows, out_q, out_s = _q8_out(x.shape, dim, gs, x.device, out_q, out_s)
    _bind(x)
    rc = _lib.load().v7g_rmsnorm_quantize(out_q.data_ptr(), out_s.data_ptr(), x.data_ptr(), weight.data_ptr(), rows,
                                          dim, int(gs), float(eps))
    _lib.check(rc, "rmsnorm_quantize")
    return out_q, out_s


def add_rmsnorm_quantize(residual: torch.Tensor, add: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                         gs: int = 64, out_q: torch.Tensor | None = None, out_s: torch.Tensor | None = None):
    """residual += add (in place), then RMSNorm -> Q8 of the updated rows: returns (codes, scales)."""
    for t, n in ((residual, "residual"), (add, "add"), (weight, "weight")):
        _need(t, torch.float32, n)
    dim = residual.shape[-1]
    if add.shape != residual.shape or weight.numel() != dim:
        raise ValueError("shape mismatch: add must match residual, weight must be [dim]")
    rows, out_q, out_s = _q8_out(residual.shape, dim, gs, residual.device, out_q, out_s)
    _bind(residual)
    rc = _lib.load().v7g_add_rmsnorm_quantize(out_q.data_ptr(), out_s.data_ptr(), residual.data_ptr(), add.data_ptr(),
                                              weight.data_ptr(), rows, dim, int(gs), float(eps))
    _lib.check(rc, "add_rmsnorm_quantize")
    return out_q, out_s


def add_inplace(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """x += y elementwise (v7s_add_inplace); returns x."""
    _need(x, torch.float32, "x")
    _need(y, torch.float32, "y")
    if x.shape != y.shape:
        raise ValueError("x and y must have the same shape")
    _bind(x)
    _lib.check(_lib.load().v7g_add_inplace(x.data_ptr(), y.data_ptr(), x.numel()), "add_inplace")
    return x


def _heads_view(buf: torch.Tensor, name: str):
    """[T, H, D] view with unit stride inside a token's heads; returns (T, H, D, token_stride)."""
    if buf.dim() != 3:
        raise ValueError(f"{name} must be [tokens, heads, head_dim]")
    T, H, D = buf.shape
    if buf.stride(2) != 1 or buf.stride(1) != D:
        raise ValueError(f"{name}: heads of one token must be contiguous")
    return T, H, D, buf.stride(0)


def _tables(cos_table: torch.Tensor, sin_table: torch.Tensor) -> None:
    for t, n in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _need(t, torch.float32, n)
    if cos_table.dim() != 2 or sin_table.shape != cos_table.shape:
        raise ValueError("cos_table and sin_table must both be [positions, rope_max_dim]")


def _head_weight(w: torch.Tensor, D: int, name: str) -> None:
    _need(w, torch.float32, name)
    if w.numel() != D:
        raise ValueError(f"{name} must hold head_dim = {D} floats")


def _positions(positions, T, device):
    if positions is None:
        return 0
    _need(positions, torch.int32, "positions")
    if positions.numel() != T:
        raise ValueError("positions must hold one int32 per token")
    return positions.data_ptr()


def rmsnorm_rope_heads(buf: torch.Tensor, norm_weight: torch.Tensor, cos_table: torch.Tensor,
                       sin_table: torch.Tensor, positions: torch.Tensor | None = None, pos0: int = 0,
                       eps: float = 1e-6) -> torch.Tensor:
    """In-place per-head RMSNorm + RoPE of buf [T, H, D] (token stride free); tables [P, rope_max_dim]."""
    _need(buf, torch.float32, "buf", contiguous=False)
    _tables(cos_table, sin_table)
    T, H, D, ts = _heads_view(buf, "buf")
    _head_weight(norm_weight, D, "norm_weight")
    _bind(buf)
    rc = _lib.load().v7g_rmsnorm_rope_heads(buf.data_ptr(), T, ts, H, D, norm_weight.data_ptr(),
                                            cos_table.data_ptr(), sin_table.data_ptr(),
                                            _positions(positions, T, buf.device), int(pos0), cos_table.shape[-1],
                                            cos_table.shape[0], float(eps))
    _lib.check(rc, "rmsnorm_rope_heads")
    return buf


def qk_rmsnorm_rope(q: torch.Tensor, k: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                    cos_table: torch.Tensor, sin_table: torch.Tensor, positions: torch.Tensor | None = None,
                    pos0: int = 0, eps: float = 1e-6, k_cache: torch.Tensor | None = None,
                    keep_k_f32: bool = True) -> None:
    """In-place RMSNorm+RoPE of Q [T, Hq, D] and K [T, Hk, D] in one launch.

    With k_cache (float16 [T, Hk, D], heads of a token contiguous, token stride free), the rotated K heads
    are also written there as binary16 (v7s_kv_pack_f16 fused); keep_k_f32=False leaves K's f32 storage
    untouched."""
    for t, n in ((q, "q"), (k, "k")):
        _need(t, torch.float32, n, contiguous=False)
    _tables(cos_table, sin_table)
    T, Hq, D, qs = _heads_view(q, "q")
    Tk, Hk, Dk, ks = _heads_view(k, "k")
    if Tk != T or Dk != D:
        raise ValueError("q and k must have the same tokens and head_dim")
    _head_weight(q_norm_weight, D, "q_norm_weight")
    _head_weight(k_norm_weight, D, "k_norm_weight")
    _bind(q)
    if k_cache is None:
        rc = _lib.load().v7g_qk_rmsnorm_rope(q.data_ptr(), qs, Hq, q_norm_weight.data_ptr(), k.data_ptr(), ks, Hk,
                                             k_norm_weight.data_ptr(), T, D, cos_table.data_ptr(),
                                             sin_table.data_ptr(), _positions(positions, T, q.device), int(pos0),
                                             cos_table.shape[-1], cos_table.shape[0], float(eps))
        _lib.check(rc, "qk_rmsnorm_rope")
        return
    _need(k_cache, torch.float16, "k_cache", contiguous=False)
    Tc, Hc, Dc, cs = _heads_view(k_cache, "k_cache")
    if (Tc, Hc, Dc) != (T, Hk, D):
        raise ValueError("k_cache must be [tokens, kv_heads, head_dim]")
    rc = _lib.load().v7g_qk_rmsnorm_rope_kv(q.data_ptr(), qs, Hq, q_norm_weight.data_ptr(), k.data_ptr(), ks, Hk,
                                            k_norm_weight.data_ptr(), T, D, cos_table.data_ptr(),
                                            sin_table.data_ptr(), _positions(positions, T, q.device), int(pos0),
                                            cos_table.shape[-1], cos_table.shape[0], float(eps),
                                            k_cache.data_ptr(), cs, int(bool(keep_k_f32)))
    _lib.check(rc, "qk_rmsnorm_rope_kv")


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = (sigmoid(gate)*gate)*up, f32 elementwise; out may be gate (in place)."""
    _need(gate, torch.float32, "gate")
    _need(up, torch.float32, "up")
    if up.shape != gate.shape:
        raise ValueError("gate and up must have the same shape")
    if out is None:
        out = torch.empty_like(gate)
    _need(out, torch.float32, "out")
    if out.shape != gate.shape:
        raise ValueError("out must match gate")
    _bind(gate)
    rc = _lib.load().v7g_swiglu_f32(out.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel())
    _lib.check(rc, "swiglu")
    return out


def _q8_out(shape, row_len, gs, device, out_q, out_s):
    rows = 1
    for d in shape[:-1]:
        rows *= d
    spr = -(-row_len // gs)
    if out_q is None:
        out_q = torch.empty(shape, dtype=torch.int8, device=device)
    if out_s is None:
        out_s = torch.empty((rows, spr), dtype=torch.float32, device=device)
    _need(out_q, torch.int8, "out_q")
    _need(out_s, torch.float32, "out_s")
    if out_q.numel() != rows * row_len or out_s.numel() != rows * spr:
        raise ValueError("output buffers have the wrong size")
    return rows, out_q, out_s


def swiglu_q8(gate: torch.Tensor, up: torch.Tensor, gs: int = 32, out_q: torch.Tensor | None = None,
              out_s: torch.Tensor | None = None):
    """SwiGLU then Q8 block quantization per row: returns (codes int8 like gate, scales [rows, hidden/gs])."""
    _need(gate, torch.float32, "gate")
    _need(up, torch.float32, "up")
    if up.shape != gate.shape:
        raise ValueError("gate and up must have the same shape")
    hidden = gate.shape[-1]
    rows, out_q, out_s = _q8_out(gate.shape, hidden, gs, gate.device, out_q, out_s)
    _bind(gate)
    rc = _lib.load().v7g_swiglu_q8(out_q.data_ptr(), out_s.data_ptr(), gate.data_ptr(), up.data_ptr(), rows, hidden,
                                   int(gs))
    _lib.check(rc, "swiglu_q8")
    return out_q, out_s


def quantize_q8(x: torch.Tensor, gs: int = 64, out_q: torch.Tensor | None = None,
                out_s: torch.Tensor | None = None):
    """v7d_quantize per row of x [..., row_len]: returns (codes, scales [rows, ceil(row_len/gs)])."""
    _need(x, torch.float32, "x")
    row_len = x.shape[-1]
    rows, out_q, out_s = _q8_out(x.shape, row_len, gs, x.device, out_q, out_s)
    _bind(x)
    rc = _lib.load().v7g_quantize_q8(out_q.data_ptr(), out_s.data_ptr(), x.data_ptr(), rows, row_len, int(gs))
    _lib.check(rc, "quantize_q8")
    return out_q, out_s


def embedding_gather_q8(ids: torch.Tensor, table_q: torch.Tensor, table_s: torch.Tensor,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = dequant(table row ids[t]); table_q [vocab, dim] int8, table_s [vocab*dim/64] f32."""
    _need(ids, torch.int32, "ids")
    _need(table_q, torch.int8, "table_q")
    _need(table_s, torch.float32, "table_s")
    if table_q.dim() != 2:
        raise ValueError("table_q must be [vocab, dim]")
    vocab, dim = table_q.shape
    if table_s.numel() != vocab * dim // Q8_EMBED_GS:
        raise ValueError("table_s must hold vocab*dim/64 scales")
    n = ids.numel()
    if out is None:
        out = torch.empty((n, dim), dtype=torch.float32, device=ids.device)
    _need(out, torch.float32, "out")
    if out.numel() != n * dim:
        raise ValueError("out must hold [ids, dim] floats")
    _bind(ids)
    rc = _lib.load().v7g_embedding_gather_q8(out.data_ptr(), ids.data_ptr(), n, table_q.data_ptr(),
                                             table_s.data_ptr(), dim, vocab)
    _lib.check(rc, "embedding_gather_q8")
    return out


def rope_only_heads(buf: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                    positions: torch.Tensor | None = None, pos0: int = 0) -> torch.Tensor:
    """In-place RoPE (no per-head norm) of buf [T, H, D]; tables [P, rope_max_dim]."""
    _need(buf, torch.float32, "buf", contiguous=False)
    _tables(cos_table, sin_table)
    T, H, D, ts = _heads_view(buf, "buf")
    _bind(buf)
    rc = _lib.load().v7g_rope_only_heads(buf.data_ptr(), T, ts, H, D, cos_table.data_ptr(), sin_table.data_ptr(),
                                         _positions(positions, T, buf.device), int(pos0), cos_table.shape[-1],
                                         cos_table.shape[0])
    _lib.check(rc, "rope_only_heads")
    return buf


def _side(buf, norm_weight, bias, cache, keep, name):
    side = _lib.QkvSide()
    if buf is None:
        return side, None
    _need(buf, torch.float32, name, contiguous=False)
    T, H, D, ts = _heads_view(buf, name)
    side.buf, side.token_stride, side.n_heads, side.keep_f32 = buf.data_ptr(), ts, H, int(bool(keep))
    if norm_weight is not None:
        _head_weight(norm_weight, D, f"{name} norm_weight")
        side.norm_weight = norm_weight.data_ptr()
    if bias is not None:
        _need(bias, torch.float32, f"{name} bias")
        if bias.numel() != H * D:
            raise ValueError(f"{name} bias must hold heads*head_dim floats")
        side.bias = bias.data_ptr()
    if cache is not None:
        _need(cache, torch.float16, f"{name} cache", contiguous=False)
        Tc, Hc, Dc, cs = _heads_view(cache, f"{name} cache")
        if (Tc, Hc, Dc) != (T, H, D):
            raise ValueError(f"{name} cache must be [tokens, heads, head_dim]")
        side.cache, side.cache_stride = cache.data_ptr(), cs
    return side, (T, D)


def qkv_rope_stage(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None, cos_table: torch.Tensor,
                   sin_table: torch.Tensor, positions: torch.Tensor | None = None, pos0: int = 0, eps: float = 1e-6,
                   q_norm_weight=None, k_norm_weight=None, q_bias=None, k_bias=None, v_bias=None, k_cache=None,
                   v_cache=None, keep_k_f32: bool = True, keep_v_f32: bool = True) -> None:
    """The Q/K/V stage of a prefill over T tokens in one launch: bias add (optional, per side), Q and K
    RMSNorm+RoPE (norm weight given) or RoPE only, binary16 K/V cache rows (optional); all in place."""
    _tables(cos_table, sin_table)
    st = _lib.QkvStage()
    st.q, shq = _side(q, q_norm_weight, q_bias, None, True, "q")
    st.k, shk = _side(k, k_norm_weight, k_bias, k_cache, keep_k_f32, "k")
    st.v, shv = _side(v, None, v_bias, v_cache, keep_v_f32, "v")
    if shq != shk or (shv is not None and shv != shq):
        raise ValueError("q, k (and v) must have the same tokens and head_dim")
    T, D = shq
    st.n_tokens, st.head_dim = T, D
    st.cos_table, st.sin_table = cos_table.data_ptr(), sin_table.data_ptr()
    st.positions = _positions(positions, T, q.device) or None
    st.pos0, st.rope_max_dim, st.table_rows, st.eps = int(pos0), cos_table.shape[-1], cos_table.shape[0], float(eps)
    _bind(q)
    _lib.check(_lib.load().v7g_qkv_rope_stage(ctypes.addressof(st)), "qkv_rope_stage")


def kv_pack_f16(src: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """binary16 copy (round to nearest even) of src [rows, row_len] f32; row strides free (row_len % 4 == 0)."""
    _need(src, torch.float32, "src", contiguous=False)
    if src.dim() != 2 or src.stride(1) != 1:
        raise ValueError("src must be [rows, row_len] with contiguous rows")
    rows, n = src.shape
    if out is None:
        out = torch.empty((rows, n), dtype=torch.float16, device=src.device)
    _need(out, torch.float16, "out", contiguous=False)
    if out.shape != src.shape or out.stride(1) != 1:
        raise ValueError("out must be [rows, row_len] with contiguous rows")
    _bind(src)
    rc = _lib.load().v7g_kv_pack_f16(out.data_ptr(), out.stride(0), src.data_ptr(), src.stride(0), rows, n)
    _lib.check(rc, "kv_pack_f16")
    return out


def kv_pack_f16_kv(k_src: torch.Tensor, v_src: torch.Tensor, k_out: torch.Tensor | None = None,
                   v_out: torch.Tensor | None = None):
    """binary16 copies of the K and V rows [rows, row_len] (views into one fused QKV buffer: the same row
    stride) in one launch; returns (k_out, v_out)."""
    _need(k_src, torch.float32, "k_src", contiguous=False)
    _need(v_src, torch.float32, "v_src", contiguous=False)
    if k_src.dim() != 2 or k_src.stride(1) != 1 or v_src.shape != k_src.shape or v_src.stride() != k_src.stride():
        raise ValueError("k_src and v_src must be [rows, row_len] with contiguous rows and the same row stride")
    rows, n = k_src.shape
    outs = []
    for o in (k_out, v_out):
        if o is None:
            o = torch.empty((rows, n), dtype=torch.float16, device=k_src.device)
        _need(o, torch.float16, "out", contiguous=False)
        if o.shape != k_src.shape or o.stride(1) != 1:
            raise ValueError("outputs must be [rows, row_len] with contiguous rows")
        outs.append(o)
    _bind(k_src)
    rc = _lib.load().v7g_kv_pack_f16_kv(outs[0].data_ptr(), outs[0].stride(0), outs[1].data_ptr(), outs[1].stride(0),
                                        k_src.data_ptr(), v_src.data_ptr(), k_src.stride(0), rows, n)
    _lib.check(rc, "kv_pack_f16_kv")
    return outs[0], outs[1]


def rope_tables(n_pos: int, head_dim: int, rope_base: float, device="cuda", llama3: dict | None = None):
    """Device cos/sin tables [n_pos, head_dim/2] (freq_j = base^(-j/half)), built on the host.

    llama3: the Llama 3 frequency scaling (rope type 1), a dict with factor, low_freq_factor,
    high_freq_factor and original_max_position_embeddings."""
    half = head_dim // 2
    c = torch.empty((n_pos, half), dtype=torch.float32, device=device)
    s = torch.empty((n_pos, half), dtype=torch.float32, device=device)
    torch.cuda.synchronize(c.device)
    L = _lib.load()
    if llama3 is None:
        rc = L.v7g_build_rope_tables(c.data_ptr(), s.data_ptr(), n_pos, head_dim, float(rope_base))
    else:
        rc = L.v7g_build_rope_tables_llama3(c.data_ptr(), s.data_ptr(), n_pos, head_dim, float(rope_base),
                                            float(llama3["factor"]), float(llama3["low_freq_factor"]),
                                            float(llama3["high_freq_factor"]),
                                            int(llama3["original_max_position_embeddings"]))
    _lib.check(rc, "rope_tables")
    return c, s
