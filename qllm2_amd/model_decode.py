"""Token decode of a whole QLLM v11 language model on the HIP kernels, for a
continuously batched set of sequences.

Replaces the per-token forward of V11LM.generate (v11/model.py:1207-1245): the
reference runs V11LM.forward (1116-1146) on one token per step for a fixed
batch that shares one step_offset; here sequences join (admit: their prompt's
prefill) and leave (release) between steps, each keeps its own position, and a
step runs only the live rows:

  embedding rows of the tokens (the tied table, interleaved [V, dim, 2])
  -> ComplexNorm                                     (qpam_cplx_fwd)
  -> per block (v11/model.py:1038-1049), h = norm1(x) from the step before:
       x += cgu_scale * down(cgu_gate(gate(h), act(up(h))))
            (gate and up in one GEMM from h; the activation and the gate in
            one launch, qpam_cgu_mix, writing the down GEMM's input)
       x += pam_scale * PAM(norm2(x))               (DecodeEngine.layer_step:
            projection GEMM, |x| gate kernel, one decode launch, o_proj GEMM)
     each residual add fused with the norm that follows it (qpam_resid_norm:
     x updated in place, the normed rows written in the GEMM dtype)
  -> output_norm -> lm_head_proj (GEMM + bias) -> lm_head_norm
  -> tied logits Re(lm . conj(E)) (one GEMM against the interleaved table).

Every ComplexLinear runs as one real GEMM on the interleaved [n, 2 d] view of
its input with weight rows [Wr, -Wi] / [Wi, Wr] interleaved per feature, so
no layout copies sit between the kernels.  The GEMMs run in fp32 or, with
dtype=torch.bfloat16, on bf16 copies of the weights and inputs (fp32
accumulation; the residual stream, the norms' statistics and the PAM states
stay fp32).  With graphs=True a whole step (every layer and the head) is
captured once per live-count bucket and replayed.

Prefill (admit) runs the same blocks over the prompt with the fused PAM layer
forward (pam_layer.forward) and hands each layer's state to the slot pool.
The model is any module with V11LM's attribute names (embed.embed_real /
embed_imag, embed_norm, blocks[i].norm1 / cgu / cgu_scale / norm2 / pam /
pam_scale, output_norm, lm_head_proj, lm_head_norm); learned position
embeddings (use_learned_pos) are not supported.
"""

import ctypes

import torch
import torch.nn.functional as F

from . import _lib
from . import pam_layer
from . import triton_kernels as tk
from .engine import DecodeEngine

MAX_DIM = 2048  # qpam_resid_norm: a thread per four complex columns, 512 per row


def _code(t):
    return _lib.QPAM_BF16 if t.dtype == torch.bfloat16 else _lib.QPAM_F32


def _rows(t, name):
    if not (t.is_cuda and t.dim() == 3 and t.shape[2] == 2 and t.stride(2) == 1 and t.stride(1) == 2):
        raise ValueError(f"qpam {name}: expected a CUDA [n, dim, 2] tensor with contiguous rows")


def _vec(t, n, device, name, what):
    """A parameter vector the kernel reads n fp32 values from."""
    if not (t.dtype == torch.float32 and t.device == device and t.numel() == n and t.is_contiguous()):
        raise ValueError(f"qpam {name}: {what} must be a contiguous float32 tensor of {n} elements on {device}")


def resid_norm(x, scale, eps, y=None, y_scale=None, out_dtype=torch.float32):
    """The residual add and the ComplexNorm after it in one launch
    (qpam_resid_norm; V11Block.forward, v11/model.py:1045-1048, inference):
    x [n, dim, 2] fp32 is updated in place to x + y * y_scale when y
    ([n, dim, 2] fp32 or bf16; y_scale a 0-dim fp32 device tensor) is given;
    returns ComplexNorm(x; scale fp32 [dim], eps) as [n, dim, 2] in out_dtype."""
    _rows(x, "resid_norm")
    if x.dtype != torch.float32:
        raise ValueError("qpam resid_norm: x must be float32")
    n, dim = x.shape[0], x.shape[1]
    _vec(scale, dim, x.device, "resid_norm", "scale")
    out = torch.empty(n, dim, 2, device=x.device, dtype=out_dtype)
    a = _lib.ResidNormArgs()
    a.rows, a.dim, a.eps = n, dim, float(eps)
    a.x, a.ldx = x.data_ptr(), x.stride(0)
    if y is not None:
        _rows(y, "resid_norm")
        if y.shape != x.shape or y_scale is None:
            raise ValueError("qpam resid_norm: y must match x and come with y_scale")
        _vec(y_scale, 1, x.device, "resid_norm", "y_scale")
        a.y, a.y_dtype, a.ldy, a.y_scale = y.data_ptr(), _code(y), y.stride(0), y_scale.data_ptr()
    a.norm_scale = scale.data_ptr()
    a.out, a.out_dtype, a.ldo = out.data_ptr(), _code(out), out.stride(0)
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().qpam_resid_norm(ctypes.byref(a), _lib.stream_ptr(x.device)), "qpam_resid_norm")
    return out


def cgu_mix(gu, hid, bias, beta=None, phase_alpha=None, phase_beta=None, out_dtype=None):
    """ComplexGatedUnit.forward between its projections in one launch
    (qpam_cgu_mix; v11/complex_ops.py:216-220, inference): gu [n, 4 hid] (the
    gate projection's interleaved output, then the up projection's) ->
    cgu_gate(gate, act(up)) as [n, hid, 2] in out_dtype (default gu's); act
    ModReLU (bias), ModSwish (bias, beta) or the phase-modulated activation
    (bias, beta, phase_alpha, phase_beta), parameters fp32 [hid]."""
    if not (gu.is_cuda and gu.dim() == 2 and gu.shape[1] == 4 * hid and gu.stride(1) == 1):
        raise ValueError("qpam cgu_mix: expected a CUDA [n, 4 hid] tensor with contiguous rows")
    n = gu.shape[0]
    for what, t in (("bias", bias), ("beta", beta), ("phase_alpha", phase_alpha), ("phase_beta", phase_beta)):
        if t is not None:
            _vec(t, hid, gu.device, "cgu_mix", what)
    out = torch.empty(n, hid, 2, device=gu.device, dtype=out_dtype or gu.dtype)
    a = _lib.CguMixArgs()
    a.rows, a.hid = n, hid
    a.gu, a.gu_dtype, a.ldg = gu.data_ptr(), _code(gu), gu.stride(0)
    a.bias = bias.data_ptr()
    a.beta = beta.data_ptr() if beta is not None else None
    a.phase_alpha = phase_alpha.data_ptr() if phase_alpha is not None else None
    a.phase_beta = phase_beta.data_ptr() if phase_beta is not None else None
    a.out, a.out_dtype, a.ldo = out.data_ptr(), _code(out), out.stride(0)
    with torch.cuda.device(gu.device):
        _lib.check(_lib.lib().qpam_cgu_mix(ctypes.byref(a), _lib.stream_ptr(gu.device)), "qpam_cgu_mix")
    return out


def interleaved_weight(wr, wi):
    """ComplexLinear weights (out, in) -> the real [2 out, 2 in] matrix that maps
    an interleaved input row [re_0, im_0, re_1, ...] to the interleaved output."""
    return torch.stack([torch.stack([wr, -wi], -1), torch.stack([wi, wr], -1)], 1).reshape(2 * wr.shape[0], -1)


def _bias(lin):
    if getattr(lin, "bias_real", None) is None:
        return None
    return torch.stack([lin.bias_real, lin.bias_imag], 1).reshape(-1)


class ModelDecoder:
    """Decode of `model` (V11LM-shaped) for up to `n_slots` concurrent sequences."""

    MAX_GRAPHS = 64

    def __init__(self, model, n_slots, *, max_len=4096, dtype=torch.float32, graphs=False, graph_bucket=16):
        if getattr(model, "pos_embed", None) is not None:
            raise NotImplementedError("ModelDecoder: learned position embeddings (use_learned_pos) are not supported")
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("ModelDecoder: dtype must be float32 or bfloat16")
        self.model = model
        self.blocks = list(model.blocks)
        self.dtype = dtype
        self.engine = DecodeEngine([b.pam for b in self.blocks], n_slots, max_len=max_len, graphs=graphs,
                                   graph_bucket=graph_bucket, dtype=dtype)
        self.pool = self.engine.pool
        self.graph_bucket = self.engine.graph_bucket
        self._graphs = {}
        self._wver = 0
        self.refresh_weights()

    # ------------------------------------------------------------ weights
    def refresh_weights(self):
        """Rebuild the GEMM weights from the model's parameters (call after
        changing them; also refreshes the PAM layers' weights)."""
        m, dt = self.model, self.dtype
        self._graphs = {}
        self._wver += 1
        self.engine.refresh_weights()
        with torch.no_grad():
            e = torch.stack([m.embed.embed_real.weight, m.embed.embed_imag.weight], -1).float()  # [V, dim, 2]
            self.vocab, self.dim = e.shape[0], e.shape[1]
            self._embed = e.contiguous()
            self._embed_w = e.reshape(self.vocab, 2 * self.dim).to(dt).contiguous()           # logits GEMM
            self._blk = []
            if self.dim % 4 or self.dim > MAX_DIM:
                raise NotImplementedError(f"ModelDecoder: dim {self.dim} (a multiple of 4 up to {MAX_DIM})")
            prm = lambda t: t.detach().float().contiguous()
            for b in self.blocks:
                cgu = b.cgu
                act = cgu.act
                hid = cgu.gate_proj.weight_real.shape[0]
                if hid % 4:
                    raise NotImplementedError(f"ModelDecoder: CGU width {hid} (a multiple of 4)")
                w_gu = torch.cat([interleaved_weight(cgu.gate_proj.weight_real, cgu.gate_proj.weight_imag),
                                  interleaved_weight(cgu.up_proj.weight_real, cgu.up_proj.weight_imag)], 0)
                # the activation by its parameters (v11/complex_ops.py:102-143): ModReLU has a
                # bias, ModSwish a bias and beta, the phase-modulated one also phase_alpha / _beta
                phase = hasattr(act, "phase_alpha")
                self._blk.append(dict(
                    norm1=(b.norm1.scale.float().contiguous(), float(b.norm1.eps)),
                    norm2=(b.norm2.scale.float().contiguous(), float(b.norm2.eps)),
                    w_gu=w_gu.to(dt).contiguous(), hid=hid,
                    w_down=interleaved_weight(cgu.down_proj.weight_real, cgu.down_proj.weight_imag).to(dt)
                    .contiguous(),
                    act_bias=prm(act.bias),
                    act_beta=prm(act.beta) if hasattr(act, "beta") else None,
                    act_pa=prm(act.phase_alpha) if phase else None,
                    act_pb=prm(act.phase_beta) if phase else None,
                    cgu_scale=b.cgu_scale.detach().float(), pam_scale=b.pam_scale.detach().float()))
            self._norm_e = (m.embed_norm.scale.float().contiguous(), float(m.embed_norm.eps))
            self._norm_o = (m.output_norm.scale.float().contiguous(), float(m.output_norm.eps))
            self._norm_h = (m.lm_head_norm.scale.float().contiguous(), float(m.lm_head_norm.eps))
            lp = m.lm_head_proj
            self._w_head = interleaved_weight(lp.weight_real, lp.weight_imag).to(dt).contiguous()
            bh = _bias(lp)
            self._b_head = None if bh is None else bh.to(dt).contiguous()

    # ------------------------------------------------------------ pieces
    @staticmethod
    def _norm(x, p):
        return tk.fused_complex_norm(x, p[0], p[1])

    def _cgu(self, h, blk):
        """The CGU of normed rows h [n, dim, 2] in the GEMM dtype -> its output
        [n, dim, 2] in the GEMM dtype: gate and up in one GEMM, the activation
        and the gate in one launch, the down GEMM."""
        n = h.shape[0]
        gu = F.linear(h.reshape(n, -1), blk["w_gu"])                          # [n, 4 hid]: gate, up interleaved
        g = cgu_mix(gu, blk["hid"], blk["act_bias"], blk["act_beta"], blk["act_pa"], blk["act_pb"])
        return F.linear(g.view(n, -1), blk["w_down"]).view(n, self.dim, 2)

    def _head(self, h):
        """Logits [n, V] (fp32) from output-normed rows h [n, dim, 2] (GEMM dtype)."""
        n = h.shape[0]
        lm = F.linear(h.reshape(n, -1), self._w_head, self._b_head).view(n, self.dim, 2)
        lm = self._norm(lm, self._norm_h)                                      # in the GEMM dtype
        logits = F.linear(lm.reshape(n, -1), self._embed_w)                     # [n, V]
        return logits if logits.dtype == torch.float32 else logits.float()

    def _next_norm(self, li):
        """The norm after block li's PAM residual (li = -1: after the embedding norm)."""
        return self._blk[li + 1]["norm1"] if li + 1 < len(self._blk) else self._norm_o

    def _tokens(self, ids, slots):
        """Every layer and the head for the listed rows: ids [n] int64, slots [n] int32."""
        dt = self.dtype
        x = self._norm(self._embed[ids], self._norm_e)                          # fp32 residual stream
        h = resid_norm(x, *self._next_norm(-1), out_dtype=dt)
        for li, blk in enumerate(self._blk):
            h = resid_norm(x, *blk["norm2"], y=self._cgu(h, blk), y_scale=blk["cgu_scale"], out_dtype=dt)
            y = self.engine.layer_step(li, h, slots)
            h = resid_norm(x, *self._next_norm(li), y=y, y_scale=blk["pam_scale"], out_dtype=dt)
        return self._head(h)

    # ------------------------------------------------------------ slots
    @torch.no_grad()
    def prefill(self, prompt_ids):
        """The model over one prompt (ids [T]) with the fused PAM prefill:
        (logits of its last token [V], the per-layer states)."""
        ids = prompt_ids.to(self._embed.device).long().view(1, -1)
        t, dt = ids.shape[1], self.dtype
        x = self._norm(self._embed[ids[0]], self._norm_e)                       # [t, dim, 2] fp32
        h = resid_norm(x, *self._next_norm(-1), out_dtype=dt)
        states = []
        for li, (blk, b) in enumerate(zip(self._blk, self.blocks)):
            h2 = resid_norm(x, *blk["norm2"], y=self._cgu(h, blk), y_scale=blk["cgu_scale"])
            y, s = pam_layer.forward(b.pam, h2.view(1, t, self.dim, 2), None, 0)
            states.append(s)
            h = resid_norm(x, *self._next_norm(li), y=y.reshape(t, self.dim, 2).contiguous(),
                           y_scale=blk["pam_scale"], out_dtype=dt)
        return self._head(h[-1:])[0], states

    def admit(self, prompt_ids):
        """A sequence with this prompt joins: its prefill's states enter a
        slot.  Returns (slot, logits of the prompt's last token)."""
        logits, states = self.prefill(prompt_ids)
        return self.engine.admit(int(prompt_ids.numel()), states), logits

    def release(self, slot):
        self.engine.release(slot)

    def layer_state(self, layer_idx, slot):
        return self.engine.layer_state(layer_idx, slot)

    # ------------------------------------------------------------ step
    @torch.no_grad()
    def step(self, ids, slots, host_slots=None):
        """One token of each listed sequence through the whole model: ids [n]
        (the tokens, device int64), slots [n] (int32 device, distinct live
        slots).  Returns the next-token logits [n, V] (fp32; with graphs a
        view of the graph's output buffer, valid until the bucket's next step)
        and advances the positions."""
        n = ids.shape[0]
        if not self.graph_bucket:
            out = self._tokens(ids, slots)
            self.pool.advance(slots, host_slots)
            return out
        if n > self.engine.n_slots:
            raise ValueError(f"ModelDecoder: {n} rows for {self.engine.n_slots} slots")
        if host_slots is None:
            host_slots = slots.tolist()
        if self.pool.live:
            self.pool.ensure_len(max(self.pool._host_pos[s] for s in self.pool.live))
        nb = -(-n // self.graph_bucket) * self.graph_bucket
        rope = self.pool.rope.data_ptr()
        if self._graphs and next(iter(self._graphs))[1] != rope:
            self._graphs = {}
        key = (nb, rope, self._wver)
        entry = self._graphs.get(key) if n else None
        if entry is None:
            if n and nb > n:  # the padded batch eagerly first: the capture then meets only shapes already run
                ids = torch.cat([ids.long(), ids.new_zeros(nb - n, dtype=torch.long)])
                slots = torch.cat([slots.to(torch.int32), self.engine._scratch[:nb - n]])
            out = self._tokens(ids.long(), slots)[:n]
            if n:
                if len(self._graphs) >= self.MAX_GRAPHS:
                    self._graphs = {}
                self._graphs[key] = self._capture(nb)
            self.pool.advance(slots[:n], host_slots)
            return out
        entry["ids"][:n].copy_(ids)
        entry["slots"][:n].copy_(slots)
        if nb > n:
            entry["ids"][n:].zero_()
            entry["slots"][n:].copy_(self.engine._scratch[:nb - n])
        entry["graph"].replay()
        self.pool.advance(slots, host_slots)
        return entry["out"][:n]

    def _capture(self, nb):
        dev = self.pool.device
        ids = torch.zeros(nb, device=dev, dtype=torch.long)
        slots = torch.zeros(nb, device=dev, dtype=torch.int32)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._tokens(ids, slots)
        return {"graph": graph, "ids": ids, "slots": slots, "out": out}

    # ------------------------------------------------------------ sampling
    @staticmethod
    def sample(logits, temperature=1.0, top_k=0, generator=None):
        """Next tokens from logits [n, V] as V11LM.generate draws them
        (v11/model.py:1222-1236, without the repetition penalty and top-p):
        greedy when temperature is 0, else top-k filtered multinomial."""
        if temperature == 0:
            return logits.argmax(-1)
        x = logits / temperature
        if top_k > 0:
            v, _ = x.topk(min(top_k, x.shape[-1]))
            x = x.masked_fill(x < v[:, -1:], float("-inf"))
        return torch.multinomial(x.softmax(-1), 1, generator=generator).squeeze(1)
