"""Device-resident Qwen3 decoder on libythip.so (the caller of the hot path).

Mirrors the reference's Qwen3 example (example/qwen3/src/qwen3.cpp:193-516):
per layer RMSNorm -> fused qkv projection -> per-head q/k RMSNorm + RoPE with
the K/V append into the cache -> GQA causal attention -> o projection +
residual -> RMSNorm -> fused gate_up -> SwiGLU -> down projection + residual,
then the final norm and the tied LM head, greedy selection.

MI355X layout and execution:
  * weights in the model's 16-bit type (bf16 by default, fp16 with
    dtype=torch.float16; rounded with the reference's yt::bfloat16 /
    yt::float16 casts) in HBM, qkv and gate_up fused as in the example's
    load() (qwen3.cpp:326-349); norms fp32; the embedding doubles as the LM
    head unless the checkpoint has lm_head.weight; a .yt checkpoint loads
    straight into this layout (Qwen3.from_yt);
  * residual stream fp32; GEMM inputs in the 16-bit type; the o/down
    projections write fp32 straight into the residual with beta = 1 (residual
    add fused into the GEMM epilogue); logits fp32;
  * KV cache in the 16-bit type, [layers][1, kv_heads, ctx, head_dim];
  * a decode step is 5 launches per layer (the RMSNorms ride in the qkv and
    gate_up GEMV prologues, SwiGLU in the gate_up GEMV's epilogue, q/k norm + RoPE +
    cache append in the split-K attention kernel, the merge of its splits in the
    o projection's prologue; the final norm and the argmax ride in the LM
    head's) with no host-side value that changes
    between steps (token id and positions live in device memory), so it is
    captured once as a HIP graph and replayed per token.
Every arithmetic operation runs in libythip.so; torch only allocates device
memory and provides the stream / graph capture.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib, ops


class Qwen3Config:
    """Qwen3Config defaults (example/qwen3/include/qwen3.hpp:46-60)."""

    def __init__(self, hidden=1024, layers=28, vocab=151936, inter=3072, n_heads=16, n_kv=8, head_dim=128,
                 max_pos=4096, eps=1e-6, theta=1e6):
        self.hidden, self.layers, self.vocab, self.inter = hidden, layers, vocab, inter
        self.n_heads, self.n_kv, self.head_dim, self.max_pos = n_heads, n_kv, head_dim, max_pos
        self.eps, self.theta = eps, theta

    @classmethod
    def from_json(cls, path: str) -> "Qwen3Config":
        """Qwen3Config::init (example/qwen3/src/qwen3.cpp:128-159): the Hugging
        Face config.json keys, each falling back to the default when absent."""
        import json
        with open(path) as f:
            j = json.load(f)
        c = cls()
        for attr, key in (("hidden", "hidden_size"), ("layers", "num_hidden_layers"), ("vocab", "vocab_size"),
                          ("eps", "rms_norm_eps"), ("theta", "rope_theta"), ("inter", "intermediate_size"),
                          ("n_heads", "num_attention_heads"), ("n_kv", "num_key_value_heads"),
                          ("head_dim", "head_dim"), ("max_pos", "max_position_embeddings")):
            if key in j:
                setattr(c, attr, type(getattr(c, attr))(j[key]))
        return c


def hf_names(cfg, i: int | None = None) -> dict:
    """Checkpoint tensor names that Qwen3Model::load reads
    (example/qwen3/src/qwen3.cpp:318-358): the model-level ones, or layer i's."""
    if i is None:
        return {"embed": "model.embed_tokens.weight", "norm": "model.norm.weight", "lm_head": "lm_head.weight"}
    p = f"model.layers.{i}."
    return {"q": p + "self_attn.q_proj.weight", "k": p + "self_attn.k_proj.weight",
            "v": p + "self_attn.v_proj.weight", "o": p + "self_attn.o_proj.weight",
            "q_norm": p + "self_attn.q_norm.weight", "k_norm": p + "self_attn.k_norm.weight",
            "gate": p + "mlp.gate_proj.weight", "up": p + "mlp.up_proj.weight", "down": p + "mlp.down_proj.weight",
            "norm1": p + "input_layernorm.weight", "norm2": p + "post_attention_layernorm.weight"}


def weight_layout(cfg) -> list[tuple[str, tuple[int, ...]]]:
    """(name, shape) of the flat weight buffer: embed, then per layer q, k, v,
    o, q_norm, k_norm, gate, up, down, norm1, norm2, then the final norm."""
    H, I, hd = cfg.hidden, cfg.inter, cfg.head_dim
    out = [("embed", (cfg.vocab, H))]
    for i in range(cfg.layers):
        out += [(f"{i}.q", (cfg.n_heads * hd, H)), (f"{i}.k", (cfg.n_kv * hd, H)), (f"{i}.v", (cfg.n_kv * hd, H)),
                (f"{i}.o", (H, cfg.n_heads * hd)), (f"{i}.q_norm", (hd,)), (f"{i}.k_norm", (hd,)),
                (f"{i}.gate", (I, H)), (f"{i}.up", (I, H)), (f"{i}.down", (H, I)),
                (f"{i}.norm1", (H,)), (f"{i}.norm2", (H,))]
    out.append(("norm", (H,)))
    return out


def rope_tables(dim: int, max_len: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """RoPECache::precompute tables built by libythip on the host."""
    c = np.empty((max_len, dim), np.float32)
    s = np.empty((max_len, dim), np.float32)
    _lib.check(_lib.lib().ythip_rope_tables(dim, max_len, float(theta), c.ctypes.data, s.ctypes.data),
               "ythip_rope_tables")
    return c, s


class Qwen3:
    """Greedy batch-1 generation on one GPU."""

    def __init__(self, cfg: Qwen3Config, weights, device="cuda", max_ctx: int | None = None,
                 max_prompt: int = 512, fused: bool = True, dtype: torch.dtype = torch.bfloat16,
                 max_tokens: int = 4096):
        """max_ctx: rows of the ring KV cache (default max_position_embeddings, the
        size the reference's KVCache::init gives it, qwen3.cpp:415-421; a smaller
        ring saves memory and wraps earlier by the same rules). max_tokens:
        history capacity, the most tokens one generate() call returns."""
        if dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("the decoder runs its matrices, activations and KV cache in bfloat16 or float16")
        self.cfg = cfg
        self.dtype = dtype  # matrices, GEMM inputs and KV cache; residual, norms and logits stay fp32
        self.fused = fused  # decode step with the fused GEMV prologues (same bits as the unfused path)
        self.dev = torch.device(device)
        self.max_ctx = min(cfg.max_pos, max_ctx or cfg.max_pos)
        self.max_prompt = max_prompt
        self.max_tokens = max_tokens
        self._upload(weights)
        self._alloc()
        self.graph = None
        self.prefill_graphs = {}  # prompt length -> captured prefill

    # ---------------------------------------------------------------- weights
    def _upload(self, weights) -> None:
        """weights: flat fp32 array (numpy or torch) in weight_layout order, a
        dict name -> tensor, or the path of a .yt checkpoint (see _load_yt).
        Matrices become the model's 16-bit type, norms stay fp32."""
        cfg, dev = self.cfg, self.dev
        if isinstance(weights, (str, bytes)) or hasattr(weights, "__fspath__"):
            self._load_yt(weights)
            return
        lay = weight_layout(cfg)
        if isinstance(weights, dict):
            get = lambda name, shp: torch.as_tensor(weights[name]).reshape(shp)
        else:
            flat = torch.as_tensor(weights)
            offs = {}
            o = 0
            for name, shp in lay:
                n = int(np.prod(shp))
                offs[name] = (o, n)
                o += n
            if flat.numel() != o:
                raise ValueError(f"weight buffer has {flat.numel()} values, the layout needs {o}")
            get = lambda name, shp: flat[offs[name][0]:offs[name][0] + offs[name][1]].reshape(shp)
        code = _lib.BF16 if self.dtype == torch.bfloat16 else _lib.F16

        def bf(t):
            # fp32 -> 16-bit on the host with the reference's cast (yt::bfloat16 / yt::float16)
            src = np.ascontiguousarray(t.detach().cpu().numpy(), dtype=np.float32)
            bits = np.empty(src.shape, np.uint16)
            _lib.check(_lib.lib().ythip_convert_host(_lib.F32, code, src.ctypes.data, bits.ctypes.data, src.size),
                       "ythip_convert_host")
            return torch.from_numpy(bits.view(np.int16)).view(self.dtype).to(dev)
        f32 = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
        self.embed = bf(get("embed", (cfg.vocab, cfg.hidden)))
        self.layers = []
        for i in range(cfg.layers):
            shp = dict(lay)
            qkv = torch.cat([get(f"{i}.q", shp[f"{i}.q"]), get(f"{i}.k", shp[f"{i}.k"]),
                             get(f"{i}.v", shp[f"{i}.v"])], 0)
            gu = torch.cat([get(f"{i}.gate", shp[f"{i}.gate"]), get(f"{i}.up", shp[f"{i}.up"])], 0)
            self.layers.append(dict(
                qkv=bf(qkv), o=bf(get(f"{i}.o", shp[f"{i}.o"])), gu=bf(gu), down=bf(get(f"{i}.down", shp[f"{i}.down"])),
                qn=f32(get(f"{i}.q_norm", shp[f"{i}.q_norm"])), kn=f32(get(f"{i}.k_norm", shp[f"{i}.k_norm"])),
                n1=f32(get(f"{i}.norm1", shp[f"{i}.norm1"])), n2=f32(get(f"{i}.norm2", shp[f"{i}.norm2"]))))
        self.fnorm = f32(get("norm", (cfg.hidden,)))
        self.lm_head = self.embed  # tied (Qwen3ForCausalLM::forward, qwen3.cpp:453-456)
        self._rope()

    def _rope(self) -> None:
        c, s = rope_tables(self.cfg.head_dim, self.cfg.max_pos, self.cfg.theta)
        self.cos = torch.from_numpy(c).to(self.dev)
        self.sin = torch.from_numpy(s).to(self.dev)

    def _load_yt(self, path) -> None:
        """Qwen3Model::load + Qwen3ForCausalLM::load (example/qwen3/src/qwen3.cpp:
        304-363, 424-431) from a .yt checkpoint, straight into the device
        layout: q/k/v land in the row blocks of the fused qkv weight and
        gate/up in gate_up (the example's concat, 326-349, without a copy);
        matrices are stored in the model's 16-bit type (converted with the
        reference's cast when the file holds another float type), norms as fp32. lm_head.weight is
        used when present, else the embedding (tied). Unlike the example, a
        missing tensor is an error rather than an empty weight."""
        from . import io as ytio
        cfg, dev = self.cfg, self.dev
        H, I, hd, nh, nkv = cfg.hidden, cfg.inter, cfg.head_dim, cfg.n_heads, cfg.n_kv
        f = ytio.YTensorIO()
        if not f.open(str(path), ytio.Read):
            raise FileNotFoundError(f"cannot open {path} as a .yt checkpoint")
        try:
            names = set(f.getTensorNames())
            bf, fp = self.dtype, torch.float32
            top = hf_names(cfg)
            need = [top["embed"], top["norm"]] + [n for i in range(cfg.layers) for n in hf_names(cfg, i).values()]
            missing = [n for n in need if n not in names]
            if missing:
                raise KeyError(f"{path}: {len(missing)} tensors missing, first {missing[:3]}")
            plan = []
            self.embed = torch.empty((cfg.vocab, H), dtype=bf, device=dev)
            plan.append((top["embed"], self.embed))
            self.layers = []
            for i in range(cfg.layers):
                n = hf_names(cfg, i)
                L = dict(qkv=torch.empty(((nh + 2 * nkv) * hd, H), dtype=bf, device=dev),
                         o=torch.empty((H, nh * hd), dtype=bf, device=dev),
                         gu=torch.empty((2 * I, H), dtype=bf, device=dev),
                         down=torch.empty((H, I), dtype=bf, device=dev),
                         qn=torch.empty((hd,), dtype=fp, device=dev), kn=torch.empty((hd,), dtype=fp, device=dev),
                         n1=torch.empty((H,), dtype=fp, device=dev), n2=torch.empty((H,), dtype=fp, device=dev))
                plan += [(n["q"], L["qkv"][:nh * hd]), (n["k"], L["qkv"][nh * hd:(nh + nkv) * hd]),
                         (n["v"], L["qkv"][(nh + nkv) * hd:]), (n["o"], L["o"]),
                         (n["gate"], L["gu"][:I]), (n["up"], L["gu"][I:]), (n["down"], L["down"]),
                         (n["q_norm"], L["qn"]), (n["k_norm"], L["kn"]),
                         (n["norm1"], L["n1"]), (n["norm2"], L["n2"])]
                self.layers.append(L)
            self.fnorm = torch.empty((H,), dtype=fp, device=dev)
            plan.append((top["norm"], self.fnorm))
            if top["lm_head"] in names:
                self.lm_head = torch.empty((cfg.vocab, H), dtype=bf, device=dev)
                plan.append((top["lm_head"], self.lm_head))
            else:
                self.lm_head = self.embed
            for name, dst in plan:
                shp = f.getTensorInfo(name).shape
                if int(np.prod(shp)) != dst.numel() or (len(shp) == 2 and tuple(shp) != tuple(dst.shape)):
                    raise ValueError(f"{path}: '{name}' has shape {shp}, the model expects {tuple(dst.shape)}")
            f.load_many(plan)
        finally:
            f.close()
        self._rope()

    @classmethod
    def from_yt(cls, model_dir_or_file: str, cfg: Qwen3Config | None = None, **kw) -> "Qwen3":
        """Qwen3ForCausalLM::init + load: `cfg` from `<dir>/config.json` when a
        directory is given (Qwen3Config::init) and the weights from
        `<dir>/model.yt`, or from the given .yt file with `cfg` (default shape)."""
        import os
        path = model_dir_or_file
        if os.path.isdir(path):
            if cfg is None and os.path.exists(os.path.join(path, "config.json")):
                cfg = Qwen3Config.from_json(os.path.join(path, "config.json"))
            path = os.path.join(path, "model.yt")
        return cls(cfg or Qwen3Config(), path, **kw)

    def _alloc(self) -> None:
        cfg, dev, P = self.cfg, self.dev, self.max_prompt
        H, nh, nkv, hd, I = cfg.hidden, cfg.n_heads, cfg.n_kv, cfg.head_dim, cfg.inter
        bf, f32 = self.dtype, torch.float32
        self.x = torch.empty((P, H), dtype=f32, device=dev)
        self.h = torch.empty((P, H), dtype=bf, device=dev)
        self.qkv = torch.empty((P, (nh + 2 * nkv) * hd), dtype=bf, device=dev)
        self.q = torch.empty((1, nh, P, hd), dtype=bf, device=dev)
        self.attn = torch.empty((P, nh * hd), dtype=bf, device=dev)
        self.gu = torch.empty((P, 2 * I), dtype=bf, device=dev)
        self.act = torch.empty((P, I), dtype=bf, device=dev)
        self.kc = torch.zeros((cfg.layers, 1, nkv, self.max_ctx, hd), dtype=bf, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.hf = torch.empty((1, H), dtype=bf, device=dev)
        self.logits = torch.empty((1, cfg.vocab), dtype=f32, device=dev)
        self.ids = torch.zeros((P,), dtype=torch.int32, device=dev)
        self.token = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.history = torch.zeros((self.max_tokens,), dtype=torch.int32, device=dev)
        # decode-state record (ring cache bookkeeping, include/ythip.h); `total`
        # mirrors its TOTAL on the host between calls
        self.state = ops.decode_state(0, self.max_ctx, cfg.max_pos, history=self.max_tokens, device=dev)
        self.total = 0
        self.mask = None  # bool mask of a prefill into a full ring (get_mask, qwen3.cpp:104-126)
        self.ws = torch.empty((ops.decode_workspace_bytes(1, nh, self.max_ctx, hd),), dtype=torch.uint8, device=dev)
        self.qd = torch.empty((1, nh, 1, hd), dtype=bf, device=dev)  # decode query
        self.amax = torch.empty((2 * ((cfg.vocab + 15) // 16),), dtype=f32, device=dev)  # LM-head tile maxima

    # ------------------------------------------------------------------ steps
    def _attn_view(self, S: int) -> torch.Tensor:
        """[1, nh, S, hd] view whose memory is attn[S, nh*hd] (no permute copy)."""
        nh, hd = self.cfg.n_heads, self.cfg.head_dim
        return self.attn[:S].view(S, nh, hd).permute(1, 0, 2).unsqueeze(0)

    def _layer(self, i: int, S: int, decode: bool, pre: dict | None = None) -> None:
        """Layer i on S rows. Decode: one token at the decode-state record's
        RoPE row / cache slot. Prefill: `pre` gives the RoPE start, the first
        cache row of the ring write, the keys visible after the append and the
        mask (None = causal over physical rows; a bool mask once the ring is
        full, as get_mask builds it)."""
        cfg, L = self.cfg, self.layers[i]
        nh, nkv, hd = cfg.n_heads, cfg.n_kv, cfg.head_dim
        x, h = self.x[:S], self.h[:S]
        kc, vc = self.kc[i], self.vc[i]
        if decode and self.fused:
            self._layer_decode_fused(i)
            return
        ops.rms_norm(x, L["n1"], cfg.eps, out=h)
        ops.gemm(h, L["qkv"].t(), self.qkv[:S])
        if decode:
            qv = self.qd
            ops.rms_norm_rope(self.qkv[:S].view(1, S, -1), nh, nkv, hd, L["qn"], L["kn"], cfg.eps, self.cos, self.sin,
                              q_out=qv, k_out=kc, v_out=vc, dev_state=self.state)
            kv_len = self.state[ops.ST_KV_LEN:ops.ST_KV_LEN + 1]
            ops.decode_attention(qv.view(1, nh, hd), kc, vc, kv_len=kv_len,
                                 out=self.attn[:1].view(1, nh, hd), workspace=self.ws)
        else:
            qv = self.q[:, :, :S, :]
            ops.rms_norm_rope(self.qkv[:S].view(1, S, -1), nh, nkv, hd, L["qn"], L["kn"], cfg.eps, self.cos, self.sin,
                              pos0=pre["start"], q_out=qv, k_out=kc, v_out=vc, cache_pos=pre["row"])
            n = pre["kv_len"]
            ops.scaled_dot_product_attention(qv, kc[:, :, :n], vc[:, :, :n], 0.0,
                                             mask="causal" if pre["mask"] is None else pre["mask"],
                                             out=self._attn_view(S))
        ops.gemm(self.attn[:S], L["o"].t(), x, beta=1.0)          # x += attn . Wo^T
        ops.rms_norm(x, L["n2"], cfg.eps, out=h)
        ops.gemm(h, L["gu"].t(), self.gu[:S])
        ops.silu_mul(self.gu[:S], out=self.act[:S])
        ops.gemm(self.act[:S], L["down"].t(), x, beta=1.0)        # x += act . Wdown^T

    def _layer_decode_fused(self, i: int) -> None:
        """One token through layer i in 5 launches: the RMSNorms ride in the
        qkv / gate_up GEMV prologues, SwiGLU in the gate_up GEMV's epilogue (each
        activation computed once, by the workgroup that owns its gate and up
        rows), the q/k norm + RoPE and cache append in the split-K attention
        kernel, and the merge of the splits in the o projection's prologue."""
        cfg, L = self.cfg, self.layers[i]
        nh, nkv, hd = cfg.n_heads, cfg.n_kv, cfg.head_dim
        x = self.x[:1]
        kc, vc = self.kc[i], self.vc[i]
        ops.gemv_fused(x, L["qkv"], self.qkv[:1], "rmsnorm", L["n1"], cfg.eps)
        # q/k norm + RoPE, the K/V append and split-K attention in one launch
        # (partials in the workspace), then the merge of the splits as the o
        # projection's prologue
        ops.decode_attention_rope(self.qkv[:1], nh, nkv, hd, L["qn"], L["kn"], cfg.eps, self.cos, self.sin,
                                  self.state, kc, vc, None, self.ws)
        ops.gemv_attn_merge(self.ws, 1, nh, hd, self.max_ctx, L["o"], x, beta=1.0, dev_state=self.state)  # x += attn . Wo^T
        ops.gemv_swiglu(x, L["gu"], self.act[:1], "rmsnorm", L["n2"], cfg.eps)    # act = swiglu(norm(x) . Wgu^T)
        ops.gemv_fused(self.act[:1], L["down"], x, beta=1.0)                      # x += act . Wdown^T

    def _head(self, S: int) -> None:
        if S == 1 and self.fused:
            # final norm + tied LM head + per-tile argmax in one launch, then the pick
            ops.gemv_fused(self.x[:1], self.lm_head, self.logits, "rmsnorm", self.fnorm, self.cfg.eps,
                           argmax_parts=self.amax)
            ops.argmax_finish(self.amax, self.amax.numel() // 2, self.token, self.history, self.state)
            return
        ops.rms_norm(self.x[S - 1:S], self.fnorm, self.cfg.eps, out=self.hf)
        ops.gemm(self.hf, self.lm_head.t(), self.logits)           # LM head (tied by default), fp32 logits
        ops.argmax_step(self.logits, self.token, self.history, self.state)

    def _prefill_body(self, P: int, pre: dict) -> None:
        ops.embedding(self.embed, self.ids[:P], self.x[:P])
        for i in range(self.cfg.layers):
            self._layer(i, P, decode=False, pre=pre)
        self._head(P)

    def _prefill_plan(self, P: int, t0: int) -> dict:
        """Where a P-token prompt goes when t0 tokens are already in the ring:
        the RoPE start (Qwen3Model::forward, qwen3.cpp:365-375), the first cache
        row (KVCache::append, 70-88), the keys visible after the append and the
        mask -- causal over physical rows while the ring has not wrapped, else
        get_mask's logical-order mask (104-126)."""
        ring, max_pos = self.max_ctx, self.cfg.max_pos
        cur = min(t0, ring)
        start = t0 if t0 > 0 else 0
        if start + P > max_pos:
            start = cur
            if start + P > max_pos:
                start = 0
        kv_len = min(cur + P, ring)
        mask = None
        if t0 + P > ring:  # full after the append: keys in logical order (ki - write_pos) mod ring
            wp = (t0 + P) % ring
            ki = np.arange(kv_len)[None, :]
            qi = np.arange(P)[:, None]
            vis = ((ki - wp + ring) % ring) <= (kv_len - P) + qi
            mask = torch.from_numpy(np.ascontiguousarray(vis, dtype=np.uint8)).to(self.dev)
        return {"start": start, "row": t0 % ring, "kv_len": kv_len, "mask": mask}

    def prefill(self, prompt, use_graph: bool = False, reset: bool = True) -> None:
        """Run the prompt; the first generated token lands in history[0].

        reset=False continues over the tokens already in the KV cache (a new
        turn, as a second Qwen3ForCausalLM::generate call does): RoPE rows,
        cache rows and the mask follow the reference's ring rules. With
        use_graph a fresh prompt's launches (embedding, every layer, head) are
        captured once per prompt length as a HIP graph and replayed: the token
        ids and the decode state are device buffers written before the replay,
        so one capture serves every prompt of that length with the eager
        path's bits (a continued prompt runs eagerly)."""
        P = len(prompt)
        ids = np.asarray(prompt, dtype=np.int64)
        if P == 0 or P > self.max_prompt or P > self.max_ctx or P > self.cfg.max_pos:
            raise ValueError(f"prompt of {P} tokens: need 1 <= P <= max_prompt={self.max_prompt}, "
                             f"max_ctx={self.max_ctx}, max_pos={self.cfg.max_pos}")
        if ids.min() < 0 or ids.max() >= self.cfg.vocab:
            raise ValueError(f"token ids must lie in [0, {self.cfg.vocab})")
        t0 = 0 if reset else self.total
        pre = self._prefill_plan(P, t0)
        self.ids[:P].copy_(torch.from_numpy(ids.astype(np.int32)))
        # the head's argmax counts the last prompt token as written: TOTAL = t0 + P after it
        ops.decode_state(t0 + P - 1, self.max_ctx, self.cfg.max_pos, history=self.max_tokens, out=self.state)
        if use_graph and t0 == 0:
            g = self.prefill_graphs.get(P)
            if g is None:
                g = self.prefill_graphs[P] = self._capture(lambda: self._prefill_body(P, pre))
            g.replay()
        else:
            self._prefill_body(P, pre)
        self.prompt_len = P
        self.total = t0 + P

    def _decode_step(self) -> None:
        ops.embedding(self.embed, self.token, self.x[:1])
        for i in range(self.cfg.layers):
            self._layer(i, 1, decode=True)
        self._head(1)

    @staticmethod
    def _capture(fn) -> "torch.cuda.CUDAGraph":
        """Record fn's launches as a HIP graph (nothing executes while capturing)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        return g

    def capture(self) -> None:
        """Capture one decode step as a HIP graph (replayed per token)."""
        self.graph = self._capture(self._decode_step)

    def generate(self, prompt, n_tokens: int, use_graph: bool = True, reset: bool = True) -> np.ndarray:
        """Greedy: prompt forward, then n_tokens - 1 decode steps. Returns the tokens.
        use_graph replays captured graphs for both (one prefill graph per prompt length).
        reset=False keeps the KV cache of the previous calls (multi-turn, as the
        reference's generate does); the ring wraps once more than max_ctx
        tokens were written."""
        if not 1 <= n_tokens <= self.max_tokens:
            raise ValueError(f"n_tokens={n_tokens}: this model's history holds 1..{self.max_tokens} tokens")
        self.prefill(prompt, use_graph=use_graph, reset=reset)
        if use_graph and self.graph is None:
            # capturing does not execute the step; state is untouched
            self.capture()
        for _ in range(n_tokens - 1):
            if use_graph:
                self.graph.replay()
            else:
                self._decode_step()
        torch.cuda.synchronize()
        self.total += n_tokens - 1
        self.check_state()
        return self.history[:n_tokens].cpu().numpy()

    def check_state(self) -> None:
        """Raise if a kernel flagged an out-of-range cache row, RoPE row or
        history entry in the decode-state record (it never accesses them)."""
        st = self.state.cpu().tolist()
        if st[ops.ST_ERROR]:
            raise RuntimeError(f"decode state error bits {st[ops.ST_ERROR]:#x} (1 cache row, 2 RoPE row, "
                               f"4 history full): {st}")
        if st[ops.ST_TOTAL] != self.total:
            raise RuntimeError(f"decode state TOTAL {st[ops.ST_TOTAL]} != {self.total} expected")
