"""Graph-captured batch-1 decode step on the gfx950 kernels.

The step mirrors the reference's fast decode (moss_tts_lite/fast.py:123-194,
fast_native.py:222-294) on the Qwen3-shaped int4 backbone:

  embed -> 36 x [RMSNorm -> int4 q|k|v -> q/k RMSNorm + RoPE + KV write -> GQA
  attention -> int4 o (+residual) -> RMSNorm -> int4 gate|up (+SiLU*up) -> int4 down
  (+residual)] -> final RMSNorm -> bf16 head + greedy argmax -> position += 1

Differences by design: the position and the next token live in device memory, so ONE
captured graph serves every cache length (the reference captures one graph per length,
fast_native.py:369-386), and greedy decoding chains steps without a host sync.

Every launch is a plain C-ABI call on torch's current stream; the launch plan (all
pointers, sizes, workspaces) is built once, so eager steps and graph capture issue the
identical kernel sequence.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as N
from . import ops
from .model import Int4Backbone, attention_scale


class FastDecoder:
    """One decode step over an :class:`Int4Backbone` (eager or hipGraph replay)."""

    def __init__(self, model: Int4Backbone):
        self.m = model
        cfg = model.cfg
        dev = model.device
        self.dev = dev
        bf = torch.bfloat16
        self.ids = torch.zeros(1, dtype=torch.int64, device=dev)      # token fed to the step
        self.pos = torch.zeros(1, dtype=torch.int64, device=dev)      # its cache position
        self.h = torch.zeros(cfg.hidden, dtype=bf, device=dev)        # residual stream
        self.x = torch.zeros(cfg.hidden, dtype=bf, device=dev)        # normed input
        self.qkv = torch.zeros(cfg.qkv_out, dtype=bf, device=dev)
        self.q = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.attn = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.act = torch.zeros(cfg.intermediate, dtype=bf, device=dev)
        self.h_final = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.logits = torch.zeros(cfg.vocab, dtype=bf, device=dev)
        self.table_ptrs = torch.tensor([model.embed_tokens.data_ptr()], dtype=torch.int64, device=dev)
        self.vocabs = torch.tensor([cfg.vocab], dtype=torch.int64, device=dev)
        gemm_ws = max(ops.gemm_workspace_bytes(1, cfg.hidden, cfg.qkv_out, cfg.group_size),
                      ops.gemm_workspace_bytes(1, cfg.hidden, 2 * cfg.intermediate, cfg.group_size),
                      ops.gemm_workspace_bytes(1, cfg.intermediate, cfg.hidden, cfg.group_size))
        self.ws = ops.reserve_workspace(dev, gemm_ws)
        lib = N.load()
        self.attn_ws = torch.zeros(int(lib.mtl_decode_attention_workspace_bytes(cfg.n_heads, cfg.head_dim)),
                                   dtype=torch.uint8, device=dev)
        self.head_ws = torch.zeros(int(lib.mtl_head_workspace_bytes(cfg.vocab)), dtype=torch.uint8,
                                   device=dev)
        self._build_plan()
        self.graph: torch.cuda.CUDAGraph | None = None

    # -- launch plan ------------------------------------------------------------------
    def _gemm(self, x, lin, n, epilogue, resid, y):
        qw, qz, sc, perm = lin.kernel_args()
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return ("mtl_w4_gemm_fused",
                (x.data_ptr(), 1, lin.in_features, qw.data_ptr(), N.META_GPTQ, sc.data_ptr(),
                 qz.data_ptr(), p(perm), n, lin.group_size, lin.zero_offset, epilogue, p(resid),
                 y.data_ptr(), N.OUT_BF16, self.ws.data_ptr(), self.ws.numel()))

    def _layer_plan(self, li: int) -> list:
        m, cfg = self.m, self.m.cfg
        lyr = m.layers[li]
        kc, vc = m.k_cache[li], m.v_cache[li]
        scale = ctypes.c_float(attention_scale(cfg))
        eps = ctypes.c_float(cfg.eps)
        return [
            ("mtl_rmsnorm", (self.h.data_ptr(), lyr["input_layernorm"].data_ptr(),
                             self.x.data_ptr(), 1, cfg.hidden, eps)),
            self._gemm(self.x, lyr["qkv"], cfg.qkv_out, N.EPI_NONE, None, self.qkv),
            ("mtl_qk_norm_rope_kv", (self.qkv.data_ptr(), lyr["q_norm"].data_ptr(),
                                     lyr["k_norm"].data_ptr(), m.rope_cos.data_ptr(),
                                     m.rope_sin.data_ptr(), self.pos.data_ptr(), self.q.data_ptr(),
                                     kc.data_ptr(), vc.data_ptr(), cfg.n_heads, cfg.n_kv_heads,
                                     cfg.head_dim, cfg.max_seq, eps)),
            ("mtl_decode_attention", (self.q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                      self.pos.data_ptr(), self.attn.data_ptr(), cfg.n_heads,
                                      cfg.n_kv_heads, cfg.head_dim, cfg.max_seq, scale,
                                      self.attn_ws.data_ptr(), self.attn_ws.numel())),
            self._gemm(self.attn, lyr["o"], cfg.hidden, N.EPI_RESIDUAL, self.h, self.h),
            ("mtl_rmsnorm", (self.h.data_ptr(), lyr["post_attention_layernorm"].data_ptr(),
                             self.x.data_ptr(), 1, cfg.hidden, eps)),
            self._gemm(self.x, lyr["gate_up"], 2 * cfg.intermediate, N.EPI_SILU_MUL, None, self.act),
            self._gemm(self.act, lyr["down"], cfg.hidden, N.EPI_RESIDUAL, self.h, self.h),
        ]

    def _build_plan(self) -> None:
        m, cfg = self.m, self.m.cfg
        lib = N.load()
        self._embed = [("mtl_embed_sum", (self.ids.data_ptr(), 1, self.table_ptrs.data_ptr(),
                                          self.vocabs.data_ptr(), cfg.hidden, self.h.data_ptr()))]
        self._layers = [self._layer_plan(li) for li in range(cfg.n_layers)]
        self._final = [
            ("mtl_rmsnorm", (self.h.data_ptr(), m.final_norm.data_ptr(), self.h_final.data_ptr(),
                             1, cfg.hidden, ctypes.c_float(cfg.eps))),
            ("mtl_bf16_gemv_argmax", (self.h_final.data_ptr(), m.head.data_ptr(), cfg.vocab,
                                      cfg.hidden, self.logits.data_ptr(),
                                      ctypes.c_void_p(self.ids.data_ptr()),
                                      self.head_ws.data_ptr(), self.head_ws.numel())),
            ("mtl_advance_position", (ctypes.c_void_p(self.pos.data_ptr()),)),
        ]
        self._fns = {name: getattr(lib, name) for name in
                     ("mtl_rmsnorm", "mtl_w4_gemm_fused", "mtl_qk_norm_rope_kv",
                      "mtl_decode_attention", "mtl_embed_sum", "mtl_bf16_gemv_argmax",
                      "mtl_advance_position")}

    def _run(self, plan) -> None:
        stream = torch.cuda.current_stream(self.dev).cuda_stream
        for name, args in plan:
            N.check(self._fns[name](*args, stream), name)

    # -- eager pieces -----------------------------------------------------------------
    def run_layer(self, li: int) -> None:
        """One decoder layer on ``self.h`` at position ``self.pos`` (writes KV)."""
        self._run(self._layers[li])

    def run_step(self) -> None:
        """One whole decode step, eager: token ``ids`` at ``pos`` -> next token in ``ids``."""
        self._run(self._embed)
        for plan in self._layers:
            self._run(plan)
        self._run(self._final)

    # -- graph ------------------------------------------------------------------------
    def capture(self) -> None:
        """Capture the whole step once; replays advance ``pos`` and feed back the token."""
        if self.graph is not None:
            return
        saved_ids, saved_pos = self.ids.clone(), self.pos.clone()
        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            for _ in range(2):
                self.run_step()
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run_step()
        torch.cuda.synchronize(self.dev)
        self.ids.copy_(saved_ids)
        self.pos.copy_(saved_pos)
        self.graph = g

    def step(self, token: int | None = None, pos: int | None = None) -> torch.Tensor:
        """One replayed step; returns the (device) next-token buffer."""
        if self.graph is None:
            raise RuntimeError("call capture() first")
        if token is not None:
            self.ids.fill_(int(token))
        if pos is not None:
            self.pos.fill_(int(pos))
        self.graph.replay()
        return self.ids

    # -- prompt + greedy loop ---------------------------------------------------------
    def prefill(self, token_ids: torch.Tensor) -> None:
        """Fill the KV cache with a prompt, one decode step per token (eager).

        Leaves ``ids`` = greedy next token and ``pos`` = prompt length.
        """
        toks = token_ids.to(device=self.dev, dtype=torch.int64).reshape(-1)
        if toks.numel() > self.m.cfg.max_seq:
            raise ValueError("prompt longer than the KV cache")
        self.m.reset_cache()
        self.pos.zero_()
        for t in range(toks.numel()):
            self.ids.copy_(toks[t:t + 1])
            self.run_step()

    def generate(self, n_steps: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy decode ``n_steps`` tokens after :meth:`prefill`; returns them [n_steps]."""
        if self.pos.item() + n_steps > self.m.cfg.max_seq:
            raise ValueError("decode would run past the KV cache")
        out = torch.empty(n_steps, dtype=torch.int64, device=self.dev)
        for i in range(n_steps):
            if use_graph:
                self.graph.replay()
            else:
                self.run_step()
            out[i:i + 1].copy_(self.ids)
        return out
