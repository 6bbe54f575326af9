"""nanoGPT with per-head dynamic freezing, calling the SAF operators.

The prefill caller of the mixed-head attention path.  It restates the parts of
/root/reference/nanogpt/model.py that sit on that path and nothing else:
GPTConfig (:1247-1305, SAF fields only), LayerNorm (:45-54), RoPE (:57-99),
the dynamic CausalSelfAttention (freeze installers :705-772, routing cache
:846-898, pre-gathered inference weights :920-944, the fused branch of
_attend_cheap :946-1015), MLP (:1193-1207), Block (:1214-1240) and GPT
(:1312-1417, weight tying and GPT-2 init).

Differences that follow from the MI355X design:
  * every attention call of the default (fused) route goes through
    ``fused_mixed_attn`` (looked up as a module global at call time, so
    harnesses can count dispatches); with no head frozen it runs the same HIP
    flash kernel for every head.  The split route (FROZEN_ATTN_FUSED=0,
    :29-32, :1017-1061) runs the live heads through the same operator with
    no head frozen and the frozen ones through frozen_pv (dense heads) or the
    frozen-only operator (when decomposed heads are frozen, where the
    reference materialises their patterns);
  * decomposed pattern parameters (alpha, rho, z) stay fp32 whatever the model
    dtype, the convention of the reference's Qwen adapter
    (qwen/nanogpt/hybrid_prior_attention.py:128-140): z of a slow decay rounded
    to bf16 would mis-scale whole rows by ~1.6%;
  * dense patterns are stored compactly, one row per dense-frozen head, and
    addressed through pidx (the Qwen adapter's layout) instead of an
    (n_head, S, S) buffer;
  * decomposed heads whose pattern is the causal mean, an exponential decay or
    a sliding window are recognised at refresh time and run the closed-form
    scan kernel.
There is no CPU path: on a CPU tensor ``fused_mixed_attn`` raises.  The
randomisation ablations, stateful blocks, checkpoint loading and training
utilities of the reference model are outside this path.
"""
import math
import os
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from kernel import (fused_mixed_attn, decomposed_logz, classify_closed_form,  # noqa: F401
                    BAND_ROWS)
import kernel as _kernel_mod

# One mixed-head operator call for live and frozen heads (the default).
# FROZEN_ATTN_FUSED=0 selects the split route instead (nanogpt/model.py:29-32,
# :1017-1061): V projected for all heads in [live..., frozen...] order, the
# live heads through the flash kernel, the frozen ones through frozen_pv (or
# the frozen-only mixed operator when decomposed heads are frozen),
# concatenated, and c_proj applied to the matching column permutation.
_FUSED = os.environ.get("FROZEN_ATTN_FUSED", "1") != "0"
_FUSED_DISPATCH_COUNT = 0


def fused_dispatch_count():
    """Number of mixed-head attention dispatches made by this process."""
    return _FUSED_DISPATCH_COUNT


@dataclass
class GPTConfig:
    block_size: int = 1024
    vocab_size: int = 50304
    n_layer: int = 12
    n_head: int = 12
    n_embd: int = 768
    dropout: float = 0.0
    bias: bool = True
    position_encoding: str = "rope"       # "rope" | "learned_absolute"
    rope_base: float = 10000.0
    rand_attn_dynamic: bool = True
    rand_attn_prior_repr: str = "decomposed"   # "dense" | "decomposed"
    freeze_pattern_dtype: str = "float32"      # dense pattern storage dtype
    rand_seed: int = 42

    def __post_init__(self):
        if self.position_encoding not in ("learned_absolute", "rope"):
            raise ValueError("position_encoding must be 'learned_absolute' or 'rope'")
        if self.freeze_pattern_dtype not in ("float32", "bfloat16"):
            raise ValueError("freeze_pattern_dtype must be 'float32' or 'bfloat16'")
        if self.rand_attn_prior_repr not in ("dense", "decomposed"):
            raise ValueError("rand_attn_prior_repr must be 'dense' or 'decomposed'")
        if self.position_encoding == "rope" and (self.n_embd // self.n_head) % 2:
            raise ValueError("RoPE requires an even attention head dimension")


class LayerNorm(nn.Module):
    """LayerNorm with an optional bias, eps 1e-5."""

    def __init__(self, ndim, bias):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(ndim))
        self.bias = nn.Parameter(torch.zeros(ndim)) if bias else None

    def forward(self, x):
        return F.layer_norm(x, self.weight.shape, self.weight, self.bias, 1e-5)


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin):
    """Llama half-rotation RoPE on (B, H, T, D) q and k."""
    if q.size(-1) != cos.size(-1) or k.size(-1) != cos.size(-1):
        raise ValueError("RoPE cache dimension does not match Q/K head dimension")
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class RotaryEmbedding(nn.Module):
    """fp32 cos/sin cache with a bf16 copy, shared by every layer."""

    def __init__(self, dim, max_seq_len, base=10000.0):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
        freqs = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.register_buffer("cos_f32", emb.cos(), persistent=False)
        self.register_buffer("sin_f32", emb.sin(), persistent=False)
        self.register_buffer("cos_bf16", emb.cos().bfloat16(), persistent=False)
        self.register_buffer("sin_bf16", emb.sin().bfloat16(), persistent=False)

    def _apply(self, fn, recurse=True):
        # the caches keep their own dtypes (fp32 and bf16) across model.to()
        keep = (self.cos_f32, self.sin_f32)
        out = super()._apply(fn, recurse)
        dev = self.cos_f32.device
        self.cos_f32, self.sin_f32 = (t.to(device=dev) for t in keep)
        self.cos_bf16 = self.cos_f32.bfloat16()
        self.sin_bf16 = self.sin_f32.bfloat16()
        return out

    def forward(self, seq_len, dtype):
        if seq_len > self.cos_f32.size(0):
            raise ValueError("sequence length exceeds the configured RoPE cache")
        if dtype == torch.bfloat16:
            cos, sin = self.cos_bf16[:seq_len], self.sin_bf16[:seq_len]
        else:
            cos = self.cos_f32[:seq_len].to(dtype)
            sin = self.sin_f32[:seq_len].to(dtype)
        return cos.view(1, 1, seq_len, -1), sin.view(1, 1, seq_len, -1)


class CausalSelfAttention(nn.Module):
    """Multi-head causal attention whose heads can be frozen to fixed patterns."""

    _FP32_BUFFERS = ("dyn_alpha", "dyn_rho", "dyn_z")

    def __init__(self, config, layer_idx=0):
        super().__init__()
        assert config.n_embd % config.n_head == 0
        self.n_head = config.n_head
        self.n_embd = config.n_embd
        self.head_dim = config.n_embd // config.n_head
        self.layer_idx = layer_idx
        self.position_encoding = config.position_encoding
        self.q_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.bias)
        self.k_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.bias)
        self.v_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.bias)
        self.c_proj = nn.Linear(config.n_embd, config.n_embd, bias=config.bias)
        self.prior_repr = config.rand_attn_prior_repr
        self._pattern_dtype = {"float32": torch.float32,
                               "bfloat16": torch.bfloat16}[config.freeze_pattern_dtype]
        S = config.block_size
        self.block_size = S
        H = config.n_head
        self.register_buffer("dyn_frozen", torch.zeros(H, dtype=torch.bool))
        self.register_buffer("dyn_decomp", torch.zeros(H, dtype=torch.bool))
        if self.prior_repr == "decomposed":
            assert S % BAND_ROWS == 0, (
                f"rand_attn_prior_repr='decomposed' needs block_size divisible by {BAND_ROWS}")
            self.register_buffer("dyn_alpha", torch.zeros(H, S))
            self.register_buffer("dyn_rho", torch.zeros(H, S))
            self.register_buffer("dyn_z", torch.zeros(H, S))
        else:
            self.dyn_alpha = self.dyn_rho = self.dyn_z = None
        # compact dense patterns: row pattern_slot[h] of dyn_pattern
        self.register_buffer("dyn_pattern", None)
        self.register_buffer("dyn_pattern_slot", torch.full((H,), -1, dtype=torch.int32))
        self._fz_dirty = True
        self._wc_key = None
        self._ws_key = None
        # trainable-pattern owner (supplement.enable), consulted per forward
        self._patterns = None

    # -- dtype handling ---------------------------------------------------
    def _apply(self, fn, recurse=True):
        # .data: a parameter (trainable patterns) has its data swapped in place
        keep = {n: getattr(self, n).data for n in self._FP32_BUFFERS
                if getattr(self, n, None) is not None}
        out = super()._apply(fn, recurse)
        for n, old in keep.items():
            new = getattr(self, n)
            if new.dtype != torch.float32:
                # re-place the exact fp32 values on the new device
                if n in self._parameters:
                    new.data = old.to(device=new.device)
                else:
                    self._buffers[n] = old.to(device=new.device)
        # a move or cast returns the patterns contiguous: back into padded rows
        if self.dyn_pattern is not None and self.dyn_pattern.stride() != self._pattern_strides(
                self.dyn_pattern.size(0), self.dyn_pattern.dtype):
            p = self.dyn_pattern
            self.dyn_pattern = self._alloc_patterns(p.size(0), p.dtype, p.device)
            self.dyn_pattern.copy_(p)
        self._fz_dirty = True
        return out

    # -- compact dense pattern storage --------------------------------------
    def _pattern_pad(self, dtype):
        """Row padding (elements) of the compact patterns: rows S elements
        apart at a multiple of 4 KB all start on the same HBM channels, and
        the dense P.V kernel reads one 32-byte piece of each of many rows at
        once, so such pitches get 256 bytes more."""
        elem = torch.empty((), dtype=dtype).element_size()
        return 256 // elem if (self.block_size * elem) % 4096 == 0 else 0

    def _pattern_strides(self, n, dtype):
        S = self.block_size
        pitch = S + self._pattern_pad(dtype)
        return (S * pitch, pitch, 1)

    def _alloc_patterns(self, n, dtype, device):
        """Zeroed (n, S, S) pattern slots: a view of (n, S, S + pad) storage."""
        S = self.block_size
        return torch.zeros(n, S, S + self._pattern_pad(dtype), device=device, dtype=dtype)[:, :, :S]

    # -- freeze installers (nanogpt/model.py:705-772) -----------------------
    @torch.no_grad()
    def freeze_heads(self, head_idx, patterns):
        """Freeze heads to dense (T, T) patterns; they are made causal and
        row-stochastic here, once."""
        head_idx = [int(h) for h in head_idx]
        if patterns.ndim != 3 or patterns.size(-2) != patterns.size(-1):
            raise ValueError("frozen patterns must have shape (n_heads, T, T)")
        if patterns.size(0) != len(head_idx):
            raise ValueError("one frozen pattern is required per head index")
        T = patterns.size(-1)
        if T > self.block_size:
            raise ValueError("frozen pattern exceeds the configured block size")
        patterns = patterns.tril()
        patterns = patterns / patterns.sum(-1, keepdim=True).clamp_min(1e-12)
        dev = self.dyn_frozen.device
        slots = self.dyn_pattern_slot
        need = [h for h in head_idx if int(slots[h]) < 0]
        if need:
            old = self.dyn_pattern
            n_old = 0 if old is None else old.size(0)
            new = self._alloc_patterns(n_old + len(need), self._pattern_dtype if old is None else old.dtype, dev)
            if old is not None:
                new[:n_old] = old
            for i, h in enumerate(need):
                slots[h] = n_old + i
            self.dyn_pattern = new
        for j, h in enumerate(head_idx):
            s = int(slots[h])
            self.dyn_pattern[s].zero_()
            self.dyn_pattern[s, :T, :T] = patterns[j].to(dev, self.dyn_pattern.dtype)
            self.dyn_frozen[h] = True
            self.dyn_decomp[h] = False
        self._fz_dirty = True

    @torch.no_grad()
    def freeze_heads_decomposed(self, head_idx, alpha, rho, z=None):
        """Freeze heads to softmax(alpha[j] + rho[i-j]); alpha, rho: (n, T)
        logit vectors; z (the row normalisers) is derived in fp32 if absent."""
        assert self.prior_repr == "decomposed", \
            "freeze_heads_decomposed requires rand_attn_prior_repr='decomposed'"
        T = alpha.size(-1)
        dev = self.dyn_alpha.device
        idx = torch.as_tensor([int(h) for h in head_idx], dtype=torch.long, device=dev)
        a32 = alpha.to(dev, torch.float32)
        r32 = rho.to(dev, torch.float32)
        z32 = decomposed_logz(a32, r32) if z is None else z.to(dev, torch.float32)
        self.dyn_frozen[idx] = True
        self.dyn_decomp[idx] = True
        self.dyn_alpha[idx, :T] = a32
        self.dyn_rho[idx, :T] = r32
        self.dyn_z[idx, :T] = z32
        self._fz_dirty = True

    def unfreeze_heads(self, head_idx):
        for h in head_idx:
            self.dyn_frozen[int(h)] = False
            self.dyn_decomp[int(h)] = False
        self._fz_dirty = True

    # -- routing cache (nanogpt/model.py:846-898) --------------------------
    def _refresh_freeze_cache(self):
        # normal (non-inference) tensors, so a cache built under inference_mode
        # can still feed a later grad-enabled forward
        with torch.inference_mode(False), torch.no_grad():
            self._refresh_freeze_cache_impl()

    def _refresh_freeze_cache_impl(self):
        frozen = self.dyn_frozen
        dev = frozen.device
        hd = self.head_dim
        self._fz_idx = frozen.nonzero(as_tuple=True)[0]
        self._uf_idx = (~frozen).nonzero(as_tuple=True)[0]
        self._n_frozen = int(self._fz_idx.numel())
        ar = torch.arange(hd, device=dev)
        self._uf_cols = (self._uf_idx[:, None] * hd + ar).reshape(-1) if self._uf_idx.numel() else None
        dec = self.dyn_decomp & frozen
        self._fz_mask_i32 = frozen.to(torch.int32) + dec.to(torch.int32)
        self._dec_any = bool(dec.any())
        hidx = torch.zeros(self.n_head, dtype=torch.int32, device=dev)
        if self._uf_idx.numel():
            hidx[self._uf_idx] = torch.arange(self._uf_idx.numel(), dtype=torch.int32, device=dev)
        self._hidx_i32 = hidx
        self._pidx_i32 = self.dyn_pattern_slot.clamp(min=0).to(torch.int32)
        if self._dec_any:
            dec_heads = dec.nonzero(as_tuple=True)[0].tolist()
            self._closed = classify_closed_form(self.dyn_alpha, self.dyn_rho, self.dyn_z,
                                                heads=dec_heads)
        else:
            self._closed = None
        # split route: [live..., frozen...] column order and the frozen group's
        # own tables (states, pattern slots, closed forms in that order)
        fz = self._fz_idx
        self._cperm_cols = (torch.cat([self._uf_idx, fz])[:, None] * hd + ar).reshape(-1)
        self._fz_states_i32 = self._fz_mask_i32.index_select(0, fz)
        self._fz_slots_i32 = self.dyn_pattern_slot.index_select(0, fz).clamp(min=0).to(torch.int32)
        self._fz_hidx_i32 = torch.zeros(self._n_frozen, dtype=torch.int32, device=dev)
        nuf = int(self._uf_idx.numel())
        self._uf_states_i32 = torch.zeros(nuf, dtype=torch.int32, device=dev)
        self._uf_hidx_i32 = torch.arange(nuf, dtype=torch.int32, device=dev)
        if self._closed is not None:
            sel = fz.cpu().numpy()
            self._fz_closed = (self._closed[0][sel].copy(), self._closed[1][sel].copy())
        else:
            self._fz_closed = None
        self._wc_key = None
        self._ws_key = None
        self._fz_dirty = False

    def train(self, mode=True):
        self._wc_key = None
        self._ws_key = None
        return super().train(mode)

    def _split_route(self):
        """True when this call takes the split route: FROZEN_ATTN_FUSED=0 and
        some head frozen (with none frozen both routes are one flash call)."""
        if self._fz_dirty:
            self._refresh_freeze_cache()
        return not _FUSED and self._n_frozen > 0

    def _split_weight_cache(self):
        """Split route, inference: Wv[cperm], [Wq[live]; Wk[live]] and
        Wc[:, cperm] gathered once per weight version / freeze change
        (nanogpt/model.py:920-944)."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.c_proj.weight)
        key = tuple((w._version, w.data_ptr()) for w in ws)
        if self._ws_key != key:
            qw, kw, vw, cw = ws
            perm, uf = self._cperm_cols, self._uf_cols
            self._ws_v = vw.index_select(0, perm).detach()
            vb = self.v_proj.bias
            self._ws_vb = None if vb is None else vb.index_select(0, perm).detach()
            self._ws_qk = self._ws_qkb = None
            if uf is not None:
                self._ws_qk = torch.cat([qw.index_select(0, uf), kw.index_select(0, uf)]).detach()
                if self.q_proj.bias is not None:
                    self._ws_qkb = torch.cat([self.q_proj.bias.index_select(0, uf),
                                              self.k_proj.bias.index_select(0, uf)]).detach()
            self._ws_c = cw.index_select(1, perm).detach()
            self._ws_key = key
        return self._ws_v, self._ws_vb, self._ws_qk, self._ws_qkb, self._ws_c

    def split_heads(self, x, rope=None):
        """Split route (nanogpt/model.py:1017-1061): (B, T, C) head outputs in
        [live..., frozen...] order and the c_proj weight whose input columns
        match that order (None on the grad path, which applies
        linear_permuted_cols itself)."""
        if self._patterns is not None:
            raise NotImplementedError("trainable patterns run on the fused route (FROZEN_ATTN_FUSED=1)")
        B, T, C = x.size()
        nh, hd = self.n_head, self.head_dim
        nf = self._n_frozen
        nuf = nh - nf
        infer = not torch.is_grad_enabled()
        if infer:
            wv, wvb, wqk, wqkb, wc = self._split_weight_cache()
            v_all = F.linear(x, wv, wvb)
        else:
            wc = None
            v_all = _kernel_mod.linear_rows(x, self.v_proj.weight, self.v_proj.bias, self._cperm_cols)
        v_all = v_all.view(B, T, nh, hd).transpose(1, 2)
        vf = v_all[:, nuf:]
        if self._dec_any:
            # decomposed heads among the frozen: the frozen-only mixed operator
            # (dense, decomposed and closed-form kernels) over the frozen group
            fz = self._fz_idx
            yf = fused_mixed_attn(vf[:, :0], vf[:, :0], vf, self.dyn_pattern, self._fz_states_i32,
                                  self._fz_hidx_i32, self._fz_slots_i32 if self.dyn_pattern is not None else None,
                                  alpha=self.dyn_alpha.index_select(0, fz), rho=self.dyn_rho.index_select(0, fz),
                                  z=self.dyn_z.index_select(0, fz), validate=False, closed_form=self._fz_closed)
        else:
            yf = _kernel_mod.frozen_pv(self.dyn_pattern, vf, self._fz_slots_i32, T)
        if nuf == 0:
            return yf.transpose(1, 2).reshape(B, T, C), wc
        if infer:
            qk = F.linear(x, wqk, wqkb)
        else:
            qk = _kernel_mod.linear_rows2(x, self.q_proj.weight, self.k_proj.weight, self.q_proj.bias,
                                          self.k_proj.bias, self._uf_cols)
        qk = qk.view(B, T, 2, nuf, hd)
        qu, ku = qk[:, :, 0].transpose(1, 2), qk[:, :, 1].transpose(1, 2)
        if self.position_encoding == "rope":
            if rope is None:
                raise ValueError("RoPE Q/K requested without a rotary cache")
            if infer and qu.dtype in (torch.bfloat16, torch.float16):
                _kernel_mod.rope_qk_(qu, ku, *rope)
            else:
                qu, ku = apply_rotary_pos_emb(qu, ku, *rope)
        yu = fused_mixed_attn(qu, ku, v_all[:, :nuf], None, self._uf_states_i32, self._uf_hidx_i32,
                              validate=False)
        y = torch.cat([yu.transpose(1, 2), yf.transpose(1, 2)], dim=2)
        return y.reshape(B, T, C), wc

    def _infer_weight_cache(self):
        """[Wq[live]; Wk[live]; Wv] gathered once per weight version / freeze
        change, so inference runs ONE projection GEMM for Q/K of the live heads
        and V of every head (nanogpt/model.py:920-944 keeps V in its own GEMM).

        The rows are padded with zeros to a multiple of 256 (the GEMM's output
        columns past Q/K/V are never read): hipBLASLt's bf16 kernels for an
        odd multiple of 128 output columns ran 1.5x as long as for the next
        multiple of 256 (M = 16384, K = 768 on MI355X: 1920 columns 72.6 us
        against 46.5 us for 2048, 1664 columns 70.2 us against 43.6 us for
        1792), the way nanoGPT pads its vocabulary to 50304."""
        qw, kw, vw = self.q_proj.weight, self.k_proj.weight, self.v_proj.weight
        key = tuple((w._version, w.data_ptr()) for w in (qw, kw, vw))
        if self._wc_key != key:
            uf = self._uf_cols
            ws = [vw] if uf is None else [qw.index_select(0, uf), kw.index_select(0, uf), vw]
            rows = sum(w.size(0) for w in ws)
            pad = -rows % 256
            if pad:
                ws.append(vw.new_zeros(pad, vw.size(1)))
            self._wc_qkv = torch.cat(ws).detach()
            if self.q_proj.bias is None:
                self._wc_qkvb = None
            else:
                bs = [self.v_proj.bias] if uf is None else [
                    self.q_proj.bias.index_select(0, uf), self.k_proj.bias.index_select(0, uf),
                    self.v_proj.bias]
                if pad:
                    bs.append(self.v_proj.bias.new_zeros(pad))
                self._wc_qkvb = torch.cat(bs).detach()
            self._wc_key = key
        return self._wc_qkv, self._wc_qkvb

    def forward(self, x, rope=None):
        if self._split_route():
            y, wc = self.split_heads(x, rope)
            if wc is None:
                return _kernel_mod.linear_permuted_cols(y, self.c_proj.weight, self.c_proj.bias, self._cperm_cols)
            return F.linear(y, wc, self.c_proj.bias)
        return self.c_proj(self.attend(x, rope))

    # K (input features) up to which the QKV projection runs as the fused
    # GEMM + RoPE kernel (measured against the library GEMM plus the RoPE pass)
    FUSED_ROPE_MAX_K = 1024

    def _fused_rope_ok(self, x, w, wb, nqk, rope):
        return (wb is None and nqk > 0 and w.size(1) <= self.FUSED_ROPE_MAX_K
                and _kernel_mod.linear_rope_usable(x, w, nqk, self.head_dim, rope[0]))

    def head_outputs(self, x, rope=None):
        """(y, W): head outputs before c_proj and the c_proj weight whose
        input columns match their order (inference)."""
        if self._split_route():
            return self.split_heads(x, rope)
        return self.attend(x, rope), self.c_proj.weight

    def attend(self, x, rope=None):
        """The block's attention before the output projection: (B, T, C) head outputs."""
        global _FUSED_DISPATCH_COUNT
        if self._fz_dirty:
            self._refresh_freeze_cache()
        B, T, C = x.size()
        nh, hd = self.n_head, self.head_dim
        nuf = nh - self._n_frozen
        hidx = self._hidx_i32
        if torch.is_grad_enabled():
            v = self.v_proj(x).view(B, T, nh, hd).transpose(1, 2)
            if nuf == 0:
                qu = ku = v[:, :0]
            else:
                qk = _kernel_mod.linear_rows2(x, self.q_proj.weight, self.k_proj.weight,
                                              self.q_proj.bias, self.k_proj.bias, self._uf_cols)
                qk = qk.view(B, T, 2, nuf, hd)
                qu, ku = qk[:, :, 0].transpose(1, 2), qk[:, :, 1].transpose(1, 2)
                if self.position_encoding == "rope":
                    if rope is None:
                        raise ValueError("RoPE Q/K requested without a rotary cache")
                    qu, ku = apply_rotary_pos_emb(qu, ku, *rope)
        else:
            # one GEMM for live Q/K and every V; RoPE rotates Q/K in place, or
            # inside the GEMM's epilogue (linear_rope) where that kernel runs
            w, wb = self._infer_weight_cache()
            nqk = 2 * nuf * hd
            rotated = False
            if self.position_encoding == "rope" and rope is not None and self._fused_rope_ok(x, w, wb, nqk, rope):
                qkv = _kernel_mod.linear_rope(x, w, nqk, hd, *rope)
                rotated = True
            else:
                qkv = F.linear(x, w, wb)
            v = qkv[..., nqk:nqk + nh * hd].view(B, T, nh, hd).transpose(1, 2)
            if nuf == 0:
                qu = ku = v[:, :0]
            else:
                qk = qkv[..., :nqk].view(B, T, 2, nuf, hd)
                qu, ku = qk[:, :, 0].transpose(1, 2), qk[:, :, 1].transpose(1, 2)
                if self.position_encoding == "rope" and not rotated:
                    if rope is None:
                        raise ValueError("RoPE Q/K requested without a rotary cache")
                    if qu.dtype in (torch.bfloat16, torch.float16):
                        _kernel_mod.rope_qk_(qu, ku, *rope)
                    else:  # the in-place kernel is bf16 / fp16; fp32 keeps torch's rotation
                        qu, ku = apply_rotary_pos_emb(qu, ku, *rope)
        _FUSED_DISPATCH_COUNT += 1
        dec = self._dec_any
        if dec and self._patterns is not None:
            # trainable alpha / rho: z of the current parameters, no scan
            pk = self._patterns.kernel_inputs(self, T)
        elif dec:
            pk = dict(alpha=self.dyn_alpha, rho=self.dyn_rho, z=self.dyn_z, closed_form=self._closed)
        else:
            pk = dict(alpha=None, rho=None, z=None, closed_form=None)
        y = fused_mixed_attn(qu, ku, v, self.dyn_pattern, self._fz_mask_i32, hidx,
                             self._pidx_i32 if self.dyn_pattern is not None else None,
                             validate=False, **pk)
        if dec and self._patterns is not None:
            y = self._patterns.attach_gradient(self, y, v, pk["z"])
        return y.transpose(1, 2).reshape(B, T, nh * hd)


class MLP(nn.Module):

    def __init__(self, config):
        super().__init__()
        self.c_fc = nn.Linear(config.n_embd, 4 * config.n_embd, bias=config.bias)
        self.gelu = nn.GELU()
        self.c_proj = nn.Linear(4 * config.n_embd, config.n_embd, bias=config.bias)

    def forward(self, x):
        return self.c_proj(self.gelu(self.c_fc(x)))

    # K (input features) up to which the fused GEMM + GELU kernel is used: it
    # is measured faster than the library GEMM plus torch's GELU at
    # d_model 768 and slower at 2048
    FUSED_GELU_MAX_K = 1024

    def fc_gelu(self, x):
        """gelu(c_fc(x)) for the prefill path: one HIP kernel (the GELU on
        the GEMM's fp32 accumulator) when the shape allows; above that K the
        library GEMM and the HIP GELU in place on its output; else torch."""
        w = self.c_fc.weight
        exact = self.gelu.approximate == "none"
        if (self.c_fc.bias is None and exact and w.size(1) <= self.FUSED_GELU_MAX_K
                and _kernel_mod.linear_gelu_usable(x, w)):
            return _kernel_mod.linear_gelu(x, w)
        u = self.c_fc(x)
        if exact and _kernel_mod.gelu_usable(u):
            return _kernel_mod.gelu_(u)
        return self.gelu(u)


class Block(nn.Module):

    def __init__(self, config, layer_idx=0):
        super().__init__()
        self.ln_1 = LayerNorm(config.n_embd, bias=config.bias)
        self.attn = CausalSelfAttention(config, layer_idx=layer_idx)
        self.ln_2 = LayerNorm(config.n_embd, bias=config.bias)
        self.mlp = MLP(config)

    def forward(self, x, rope=None):
        x = x + self.attn(self.ln_1(x), rope=rope)
        return x + self.mlp(self.ln_2(x))


class GPT(nn.Module):

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(config.vocab_size, config.n_embd),
            wpe=nn.Embedding(config.block_size, config.n_embd),
            h=nn.ModuleList([Block(config, i) for i in range(config.n_layer)]),
            ln_f=LayerNorm(config.n_embd, bias=config.bias),
        ))
        self.rotary = (RotaryEmbedding(config.n_embd // config.n_head, config.block_size,
                                       config.rope_base)
                       if config.position_encoding == "rope" else None)
        self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.transformer.wte.weight = self.lm_head.weight
        self.apply(self._init_weights)
        for pn, p in self.named_parameters():
            if pn.endswith("c_proj.weight"):
                torch.nn.init.normal_(p, mean=0.0, std=0.02 / math.sqrt(2 * config.n_layer))
        if config.position_encoding == "rope":
            self.transformer.wpe.weight.requires_grad_(False)

    @staticmethod
    def _init_weights(module):
        if isinstance(module, nn.Linear):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                torch.nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def attn_modules(self):
        return [b.attn for b in self.transformer.h]

    def prepare_inputs(self, idx):
        _, t = idx.size()
        assert t <= self.config.block_size, \
            f"Cannot forward sequence of length {t}, block size is only {self.config.block_size}"
        x = self.transformer.wte(idx)
        if self.config.position_encoding == "learned_absolute":
            x = x + self.transformer.wpe(torch.arange(t, device=idx.device))
            return x, None
        dtype = x.dtype
        if idx.device.type == "cuda" and torch.is_autocast_enabled():
            dtype = torch.get_autocast_gpu_dtype()
        return x, self.rotary(t, dtype)

    def forward_hidden(self, idx):
        x, rope = self.prepare_inputs(idx)
        blocks = self.transformer.h
        if (x.is_cuda and not torch.is_grad_enabled()
                and x.dtype in (torch.bfloat16, torch.float16)):
            # prefill: each residual add of Block.forward runs fused with the
            # LayerNorm after it (ln_2, then the next block's ln_1 or ln_f);
            # x is the embedding output, updated in place
            # without projection biases the residual add runs inside the
            # projection GEMM (x += y W^T, one rounding) and the LayerNorm
            # after it reads x alone
            x = x.contiguous()
            x2 = x.view(-1, x.size(-1))
            ln = blocks[0].ln_1
            h = _kernel_mod.add_layernorm_(x, None, ln.weight, ln.bias)
            for i, block in enumerate(blocks):
                attn, mlp = block.attn, block.mlp
                if attn.c_proj.bias is None:
                    y, wc = attn.head_outputs(h, rope=rope)
                    x2.addmm_(y.reshape(x2.size(0), -1), wc.t())
                    h = _kernel_mod.add_layernorm_(x, None, block.ln_2.weight, block.ln_2.bias)
                else:
                    h = _kernel_mod.add_layernorm_(x, attn(h, rope=rope), block.ln_2.weight, block.ln_2.bias)
                ln = blocks[i + 1].ln_1 if i + 1 < len(blocks) else self.transformer.ln_f
                if mlp.c_proj.bias is None:
                    u = mlp.fc_gelu(h)
                    x2.addmm_(u.reshape(x2.size(0), -1), mlp.c_proj.weight.t())
                    h = _kernel_mod.add_layernorm_(x, None, ln.weight, ln.bias)
                else:
                    h = _kernel_mod.add_layernorm_(x, mlp(h), ln.weight, ln.bias)
            return h
        for block in blocks:
            x = block(x, rope=rope)
        return self.transformer.ln_f(x)

    def forward_all_positions(self, idx):
        return self.lm_head(self.forward_hidden(idx))

    def forward(self, idx):
        """Prefill: last-position logits (B, 1, vocab)."""
        x = self.forward_hidden(idx)
        return self.lm_head(x[:, -1:, :])
