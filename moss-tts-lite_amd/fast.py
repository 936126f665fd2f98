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

Five launch plans produce the same step:

* ``"strip"`` (default): five launches per layer and no cross-workgroup reduction after
  the attention.  o, gate|up and down run as the full-K strip GEMV (a workgroup owns
  16-column strips over all of K): gate|up applies SiLU*up in its epilogue and down reads
  that bf16 product, and o and down apply the residual add in their epilogue (publishing
  the sums of squares and the scattered copy of ``h`` the next RMSNorm-staged GEMV reads).
  q|k|v runs as a strip GEMV too (two strips per workgroup for GPTQ linears), handing the
  attention one "split"; ``split_k=("qkv",)`` keeps it on the split-K GEMV over the tiled
  copy instead.  The strip GEMVs sum in another order than the split-K plans', so this
  plan agrees with them to rounding, not bitwise.  It reads only the strip copies of the
  weights, so it runs on a model after ``Int4Backbone.keep_strip_copies_only()``.

* ``"staged"``: each int4 GEMV publishes only its split-K partials and the
  consumer folds the reduction in.  A 16-workgroup residual add sums the o/down
  partials into ``h``, publishes 16 block sums of squares and scatters ``h`` into the
  next GEMV's act-order input order; that GEMV applies RMSNorm while staging its input
  (norm weight pre-gathered by the same order).  The attention kernel rebuilds q/k/v
  from the q|k|v partials (q/k norm, RoPE, KV write inside), its combine scatters into
  the o projection's input order, down stages SiLU*up from the gate|up partials and the
  head applies the final norm.  8 launches per layer.
* ``"fused"``: five launches per layer.  As ``"staged"``, except that the o and down
  GEMVs reduce their split-K partials inside the kernel and apply the residual add in
  their epilogue, publishing the sums of squares and the scattered copy of ``h`` the
  next RMSNorm-staged GEMV reads.  Bitwise equal to ``"staged"``; measured slower on
  MI355X (the in-kernel cross-workgroup hand-off costs more than the separate kernel).
* ``"partials"``: the same partials hand-off, with a single-workgroup residual+RMSNorm
  kernel and a separate q/k norm+RoPE kernel (9 launches per layer).
* ``"unfused"``: each GEMV runs to completion (in-kernel reduction and epilogue).
"""
from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _native as N
from . import ops
from .gptq import QszLinear
from .model import Int4Backbone, attention_scale


def _inverse(perm: torch.Tensor | None) -> torch.Tensor | None:
    """``inv[perm[j]] = j`` (int32), or None for the identity."""
    if perm is None:
        return None
    inv = torch.empty_like(perm)
    inv[perm.long()] = torch.arange(perm.numel(), dtype=torch.int32, device=perm.device)
    return inv


def _gather(w: torch.Tensor, perm: torch.Tensor | None) -> torch.Tensor:
    return w if perm is None else w[perm.long()].contiguous()


def _check_ids(ids, limits) -> None:
    """``ValueError`` unless every id of each column lies inside its embedding table
    (``limits[c]`` rows for column c), as the reference's embedding lookups require
    (model.py:156-161). ``ids`` is ``[rows, columns]`` (host or device)."""
    t = torch.as_tensor(ids).reshape(-1, len(limits)).to("cpu", torch.int64)
    lim = torch.tensor(limits, dtype=torch.int64)
    bad = (t < 0) | (t >= lim)
    if bool(bad.any()):
        r, c = (int(v) for v in bad.nonzero()[0])
        raise ValueError(f"id {int(t[r, c])} in column {c} is outside its embedding table "
                         f"of {int(lim[c])} rows")


def _check_pos(pos: int, max_seq: int) -> int:
    pos = int(pos)
    if not 0 <= pos < max_seq:
        raise ValueError(f"position {pos} is outside the KV cache of {max_seq} positions")
    return pos


@contextlib.contextmanager
def _capturing(g: torch.cuda.CUDAGraph):
    """``torch.cuda.graph(g)`` with inference mode off. A capture registers the default
    CUDA generator's graph state, whose tensors torch creates on first use and updates in
    place at every later capture: created under inference mode (generation runs there, as
    the reference's does, fast.py:342), they would refuse a later capture outside it. The
    captured work is library launches only, so the mode changes nothing in the graph."""
    with torch.inference_mode(False), torch.cuda.graph(g):
        yield


class FastDecoder:
    """One decode step over an :class:`Int4Backbone` (eager or hipGraph replay)."""

    PLANS = ("strip", "fused", "staged", "partials", "unfused")

    def __init__(self, model: Int4Backbone, plan: str = "strip", split_k: tuple | None = None,
                 strip_geometry: dict | None = None):
        """``strip_geometry`` maps a GEMV name ("qkv", "o", "gate_up", "down") to the launch
        shape of its strip launch, ``dict(ct=, nb=, ring=, xcd_order=)`` with 0 for automatic
        (``mtl_strip_geometry``); the default is the library's automatic choice."""
        if plan not in self.PLANS:
            raise ValueError(f"plan must be one of {self.PLANS}")
        # the reference's (packed, qsz) records exist in the strip layout only
        qsz = any(isinstance(lyr[k], QszLinear) for lyr in model.layers
                  for k in ("qkv", "o", "gate_up", "down"))
        if split_k is None:
            split_k = ()
        if not set(split_k) <= {"qkv", "gate_up"} or (split_k and plan != "strip"):
            raise ValueError("split_k names GEMVs of the strip plan: 'qkv', 'gate_up'")
        if qsz and (plan != "strip" or split_k):
            raise ValueError("(packed, qsz) linears run in the strip plan with split_k=()")
        self.m = model
        self.plan = plan
        geo = dict(strip_geometry or {})
        if not set(geo) <= {"qkv", "o", "gate_up", "down"}:
            raise ValueError("strip_geometry names GEMVs: 'qkv', 'o', 'gate_up', 'down'")
        self._geom = {k: N.StripGeometry(int(v.get("ct", 0)), int(v.get("nb", 0)),
                                         int(v.get("ring", 0)), int(v.get("xcd_order", 0)))
                      for k, v in geo.items()}
        # q|k|v of GPTQ linears on the strip GEMV: two strips per workgroup unless a geometry
        # is given (measured: 1485.6 us per step against 1503.4 with one strip and 1487.8
        # on the split-K GEMV, whose tiled copy of the weight it no longer needs)
        self._qkv_geom = None
        if plan == "strip" and not qsz and "qkv" not in split_k and "qkv" not in geo and \
                all(lyr["qkv"].out_features % 32 == 0 for lyr in model.layers):
            self._qkv_geom = N.StripGeometry(2, 0, 0, 0)
        # layers whose v_proj stays bf16: q|k on the int4 strip GEMV and v on the bf16
        # GEMV, both into one fp32 "split" of the q|k|v partials the attention reads
        self.v_keep = ["v_keep" in lyr for lyr in model.layers]
        # layers whose up_proj stays bf16: the int4 gate and the bf16 up write fp32 halves
        # of the gate|up partials, an elementwise pass forms SiLU(gate) * up
        self.up_keep = ["up_keep" in lyr for lyr in model.layers]
        if (any(self.v_keep) or any(self.up_keep)) and plan != "strip":
            raise ValueError("layers with a bf16-kept v_proj or up_proj run in the strip plan")
        self.fused = plan != "unfused"
        self.strip = plan == "strip"
        # prompt rows: the q|k|v, o and down GEMMs leave their split partials, and the next
        # launch sums them (q/k norm + RoPE + KV write; residual add + the next RMSNorm)
        # (False: the GEMMs' own split-sum launches, then those launches; the same bits)
        self.fuse_split_sums = True
        # with fuse_split_sums: the norms stage x for the q|k|v and gate|up GEMMs (pair order
        # and 32-channel sums), so their workgroups copy it instead of reordering and summing
        # it (False: each GEMM stages x itself; the same bits)
        self.stage_prefill_x = True
        # strip plan: which GEMVs run as full-K strips (one "split"); the others (split_k)
        # keep the split-K kernel and hand their partials to the consumer
        self.strip_gemv = {name: self.strip and name not in split_k
                           for name in ("qkv", "o", "gate_up", "down")}
        cfg = model.cfg
        dev = model.device
        self.dev = dev
        bf = torch.bfloat16
        self._alloc_io()
        self.pos = torch.zeros(1, dtype=torch.int64, device=dev)      # its cache position
        self.h = torch.zeros(cfg.hidden, dtype=bf, device=dev)        # residual stream
        self.x = torch.zeros(cfg.hidden, dtype=bf, device=dev)        # normed input
        self.qkv = torch.zeros(cfg.qkv_out, dtype=bf, device=dev)
        self.q = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.attn = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.act = torch.zeros(cfg.intermediate, dtype=bf, device=dev)
        self.h_final = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        gemm_ws = max(ops.gemm_workspace_bytes(1, cfg.hidden, cfg.qkv_out, cfg.group_size),
                      ops.gemm_workspace_bytes(1, cfg.hidden, 2 * cfg.intermediate, cfg.group_size),
                      ops.gemm_workspace_bytes(1, cfg.intermediate, cfg.hidden, cfg.group_size))
        self.ws = ops.reserve_workspace(dev, gemm_ws)
        lib = N.load()
        self.attn_ws = torch.zeros(int(lib.mtl_decode_attention_workspace_bytes(cfg.n_heads, cfg.head_dim)),
                                   dtype=torch.uint8, device=dev)
        self.head_ws = torch.zeros(int(lib.mtl_head_workspace_bytes(cfg.vocab)), dtype=torch.uint8,
                                   device=dev)
        # fused plan: per-GEMV split-K partial buffers and the act-order input buffers
        self.splits = {name: 1 if self.strip_gemv[name] else int(lib.mtl_w4_gemm_splits(k, n))
                       for name, k, n in
                       (("qkv", cfg.hidden, cfg.qkv_out), ("o", cfg.hidden, cfg.hidden),
                        ("gate_up", cfg.hidden, 2 * cfg.intermediate),
                        ("down", cfg.intermediate, cfg.hidden))}
        cols = {"qkv": cfg.qkv_out, "o": cfg.hidden, "gate_up": 2 * cfg.intermediate,
                "down": cfg.hidden}
        self.part = {k: torch.zeros(self.splits[k] * cols[k], dtype=torch.float32, device=dev)
                     for k in cols}
        self.x_qkv = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.x_o = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.x_gu = torch.zeros(cfg.hidden, dtype=bf, device=dev)
        self.slots = torch.zeros(1024, dtype=torch.float32, device=dev)   # sum h^2 per 16 cols
        # split-K workspace of the residual GEMVs (o, down): counters stay zero between launches
        self.res_ws = torch.zeros(max(ops.gemm_workspace_bytes(1, cfg.hidden, cfg.hidden, cfg.group_size),
                                      ops.gemm_workspace_bytes(1, cfg.intermediate, cfg.hidden,
                                                               cfg.group_size)),
                                  dtype=torch.uint8, device=dev)
        self.inv_perm_o, self.inv_perm_qkv, self.inv_perm_gu = [], [], []
        self.norm_qkv, self.norm_gu = [], []      # norm weights gathered by the GEMV's perm
        for lyr in model.layers:
            self.inv_perm_o.append(_inverse(lyr["o"].perm))
            pq, pg = lyr["qkv"].perm, lyr["gate_up"].perm
            self.inv_perm_qkv.append(_inverse(pq))
            self.inv_perm_gu.append(_inverse(pg))
            self.norm_qkv.append(_gather(lyr["input_layernorm"], pq))
            self.norm_gu.append(_gather(lyr["post_attention_layernorm"], pg))
        self._build_plan()
        self.graph: torch.cuda.CUDAGraph | None = None

    def _alloc_io(self) -> None:
        """Step inputs/outputs: the token id fed in, logits and the greedy token out."""
        cfg, dev = self.m.cfg, self.m.device
        self.ids = torch.zeros(1, dtype=torch.int64, device=dev)      # token fed to the step
        self.logits = torch.zeros(cfg.vocab, dtype=torch.bfloat16, device=dev)
        self.table_ptrs = torch.tensor([self.m.embed_tokens.data_ptr()], dtype=torch.int64,
                                       device=dev)
        self.id_limits = [cfg.text_embed_rows]
        self.vocabs = torch.tensor(self.id_limits, dtype=torch.int64, device=dev)

    # -- launch plan ------------------------------------------------------------------
    def _gemm(self, x, lin, n, epilogue, resid, y, no_perm=False):
        qw, qz, sc, perm = lin.kernel_args()
        if no_perm:
            perm = None
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return ("mtl_w4_gemm_fused",
                (x.data_ptr(), 1, lin.in_features, qw.data_ptr(), N.META_GPTQ, sc.data_ptr(),
                 qz.data_ptr(), p(perm), n, lin.group_size, lin.zero_offset, epilogue, p(resid),
                 y.data_ptr(), N.OUT_BF16, self.ws.data_ptr(), self.ws.numel()))

    @staticmethod
    def _weight(lin, strip: bool):
        """``(weight, layout, metadata, zeros)`` of one int4 GEMV launch: the strip copy
        with its strip-ordered metadata (or the qsz read in place), else the split-K form."""
        qw, layout = lin.stream_weight(strip)
        if layout in (N.LAYOUT_STRIP, N.LAYOUT_STRIP_QSZ):
            sc, qz = lin.strip_meta()
        else:
            _, qz, sc, _ = lin.kernel_args()
        return qw, layout, sc, qz

    def _with_geometry(self, launch, name):
        """The launch through its ``_geom`` entry when a strip geometry is set for ``name``."""
        fn, args = launch
        layout = {"mtl_w4_gemm_partials": 13, "mtl_w4_gemm_norm_partials": 11,
                  "mtl_w4_gemm_residual": 11, "mtl_w4_gemm_norm_silu": 11}[fn]
        if name not in self._geom or args[layout] not in (N.LAYOUT_STRIP, N.LAYOUT_STRIP_QSZ):
            return launch
        return fn + "_geom", args + (ctypes.byref(self._geom[name]),)

    def _partials(self, x, xpart_name, lin, n, name):
        """Partials-only GEMV; its input is already in the weight's act-order row order."""
        qw, layout, sc, qz = self._weight(lin, self.strip_gemv[name])
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        xpart = self.part[xpart_name] if xpart_name else None
        xs = self.splits[xpart_name] if xpart_name else 0
        out = self.part[name]
        return self._with_geometry(("mtl_w4_gemm_partials",
                (p(x), p(xpart), xs, 2 * lin.in_features if xpart_name else 0, 1,
                 lin.in_features, qw.data_ptr(), sc.data_ptr(), p(qz),
                 None, n, lin.group_size,
                 lin.zero_offset, layout, out.data_ptr(), out.numel() * 4)), name)

    def _layer_plan_fused(self, li: int) -> list:
        m, cfg = self.m, self.m.cfg
        lyr = m.layers[li]
        kc, vc = m.k_cache[li], m.v_cache[li]
        scale = ctypes.c_float(attention_scale(cfg))
        eps = ctypes.c_float(cfg.eps)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        prev = self.part["down"] if li > 0 else None
        perm_qkv = lyr["qkv"].perm
        perm_gu = lyr["gate_up"].perm
        if not lyr["act_in_down_order"] and lyr["down"].perm is not None:
            raise RuntimeError("fused plan needs gate|up columns in the down input order")
        return [
            ("mtl_residual_rmsnorm", (p(prev), self.splits["down"], self.h.data_ptr(),
                                      self.h.data_ptr(), lyr["input_layernorm"].data_ptr(),
                                      self.x_qkv.data_ptr(), p(perm_qkv), cfg.hidden, eps)),
            self._partials(self.x_qkv, None, lyr["qkv"], cfg.qkv_out, "qkv"),
            ("mtl_qk_norm_rope_kv_partials", (self.part["qkv"].data_ptr(), self.splits["qkv"],
                                              lyr["q_norm"].data_ptr(), lyr["k_norm"].data_ptr(),
                                              m.rope_cos.data_ptr(), m.rope_sin.data_ptr(),
                                              self.pos.data_ptr(), self.q.data_ptr(),
                                              kc.data_ptr(), vc.data_ptr(), cfg.n_heads,
                                              cfg.n_kv_heads, cfg.head_dim, cfg.max_seq, eps)),
            ("mtl_decode_attention", (self.q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                      self.pos.data_ptr(), self.x_o.data_ptr(),
                                      p(self.inv_perm_o[li]), cfg.n_heads, cfg.n_kv_heads,
                                      cfg.head_dim, cfg.max_seq, scale, self.attn_ws.data_ptr(),
                                      self.attn_ws.numel())),
            self._partials(self.x_o, None, lyr["o"], cfg.hidden, "o"),
            ("mtl_residual_rmsnorm", (self.part["o"].data_ptr(), self.splits["o"], self.h.data_ptr(),
                                      self.h.data_ptr(), lyr["post_attention_layernorm"].data_ptr(),
                                      self.x_gu.data_ptr(), p(perm_gu), cfg.hidden, eps)),
            self._partials(self.x_gu, None, lyr["gate_up"], 2 * cfg.intermediate, "gate_up"),
            self._partials(None, "gate_up", lyr["down"], cfg.hidden, "down"),
        ]

    def _layer_plan_staged(self, li: int) -> list:
        m, cfg = self.m, self.m.cfg
        lyr = m.layers[li]
        kc, vc = m.k_cache[li], m.v_cache[li]
        scale = ctypes.c_float(attention_scale(cfg))
        eps = ctypes.c_float(cfg.eps)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        prev = self.part["down"] if li > 0 else None
        if not lyr["act_in_down_order"] and lyr["down"].perm is not None:
            raise RuntimeError("staged plan needs gate|up columns in the down input order")
        return [
            ("mtl_residual_add", (p(prev), self.splits["down"], self.h.data_ptr(),
                                  p(self.inv_perm_qkv[li]), self.x_qkv.data_ptr(),
                                  self.slots.data_ptr(), cfg.hidden)),
            self._norm_partials(self.x_qkv, self.norm_qkv[li], lyr["qkv"], cfg.qkv_out, "qkv"),
            ("mtl_decode_attention_fused", (self.part["qkv"].data_ptr(), self.splits["qkv"],
                                            lyr["q_norm"].data_ptr(), lyr["k_norm"].data_ptr(),
                                            m.rope_cos.data_ptr(), m.rope_sin.data_ptr(),
                                            kc.data_ptr(), vc.data_ptr(), self.pos.data_ptr(),
                                            self.x_o.data_ptr(), p(self.inv_perm_o[li]),
                                            cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                            cfg.max_seq, scale, eps, self.attn_ws.data_ptr(),
                                            self.attn_ws.numel())),
            self._partials(self.x_o, None, lyr["o"], cfg.hidden, "o"),
            ("mtl_residual_add", (self.part["o"].data_ptr(), self.splits["o"], self.h.data_ptr(),
                                  p(self.inv_perm_gu[li]), self.x_gu.data_ptr(),
                                  self.slots.data_ptr(), cfg.hidden)),
            self._norm_partials(self.x_gu, self.norm_gu[li], lyr["gate_up"],
                                2 * cfg.intermediate, "gate_up"),
            self._partials(None, "gate_up", lyr["down"], cfg.hidden, "down"),
        ]

    def _layer_plan_resid(self, li: int) -> list:
        """Five launches: q|k|v (RMSNorm staged), attention, o with the residual add in
        its epilogue, gate|up (RMSNorm staged), down with the residual add."""
        m, cfg = self.m, self.m.cfg
        lyr = m.layers[li]
        kc, vc = m.k_cache[li], m.v_cache[li]
        scale = ctypes.c_float(attention_scale(cfg))
        eps = ctypes.c_float(cfg.eps)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        if not lyr["act_in_down_order"] and lyr["down"].perm is not None:
            raise RuntimeError("fused plan needs gate|up columns in the down input order")
        last = li + 1 == cfg.n_layers
        plan = []
        qkv_splits = self.splits["qkv"]
        if self.v_keep[li]:   # the int4 q|k GEMV and the bf16 v_proj in one launch
            nqk = lyr["qkv"].out_features
            launches = self._with_bf16(
                self._norm_partials(self.x_qkv, self.norm_qkv[li], lyr["qkv"], nqk, "qkv",
                                    strip=True),
                lyr["input_layernorm"], lyr["v_keep"], self.part["qkv"][nqk:])
            self._keep_launches[(li, "v")] = len(launches)
            plan += launches
            qkv_splits = 1
        else:
            launch = self._norm_partials(self.x_qkv, self.norm_qkv[li], lyr["qkv"],
                                         cfg.qkv_out, "qkv")
            if self._qkv_geom is not None and launch[0] == "mtl_w4_gemm_norm_partials":
                launch = (launch[0] + "_geom", launch[1] + (ctypes.byref(self._qkv_geom),))
            plan.append(launch)
        plan += [
            ("mtl_decode_attention_fused", (self.part["qkv"].data_ptr(), qkv_splits,
                                            lyr["q_norm"].data_ptr(), lyr["k_norm"].data_ptr(),
                                            m.rope_cos.data_ptr(), m.rope_sin.data_ptr(),
                                            kc.data_ptr(), vc.data_ptr(), self.pos.data_ptr(),
                                            self.x_o.data_ptr(), p(self.inv_perm_o[li]),
                                            cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                            cfg.max_seq, scale, eps, self.attn_ws.data_ptr(),
                                            self.attn_ws.numel())),
            self._residual(self.x_o, None, lyr["o"], self.inv_perm_gu[li], self.x_gu, "o"),
        ]
        if self.up_keep[li]:   # int4 gate and bf16 up into fp32 halves; down stages SiLU*up
            inter = cfg.intermediate
            gu = self.part["gate_up"]
            launches = self._with_bf16(
                self._norm_partials(self.x_gu, self.norm_gu[li], lyr["gate_up"], inter,
                                    "gate_up", strip=True),
                lyr["post_attention_layernorm"], lyr["up_keep"], gu[inter:])
            self._keep_launches[(li, "up")] = len(launches)
            plan += launches + [
                self._residual(None, "gate_up", lyr["down"],
                               None if last else self.inv_perm_qkv[li + 1],
                               None if last else self.x_qkv, halves=True),
            ]
        elif self.strip_gemv["gate_up"]:   # SiLU*up in the epilogue; down reads the product
            plan += [
                self._norm_silu(self.x_gu, self.norm_gu[li], lyr["gate_up"]),
                self._residual(self.act, None, lyr["down"],
                               None if last else self.inv_perm_qkv[li + 1],
                               None if last else self.x_qkv),
            ]
        else:
            plan += [
                self._norm_partials(self.x_gu, self.norm_gu[li], lyr["gate_up"],
                                    2 * cfg.intermediate, "gate_up"),
                self._residual(None, "gate_up", lyr["down"],
                               None if last else self.inv_perm_qkv[li + 1],
                               None if last else self.x_qkv),
            ]
        return plan

    def _with_bf16(self, gemv, norm_w, keep, out):
        """An RMSNorm-staged int4 GEMV launch joined by the bf16-kept projection of the same
        normed h (``mtl_w4_gemm_norm_partials_bf16``: one launch where its shape applies,
        the same bits as the two); with an explicit launch geometry, the two launches."""
        eps = ctypes.c_float(self.m.cfg.eps)
        rows = ("mtl_bf16_gemv_norm", (self.h.data_ptr(), norm_w.data_ptr(), self.slots.data_ptr(),
                                       eps, keep.data_ptr(), keep.shape[0], self.m.cfg.hidden,
                                       out.data_ptr()))
        name, args = gemv
        if name != "mtl_w4_gemm_norm_partials":
            return [gemv, rows]
        return [("mtl_w4_gemm_norm_partials_bf16",
                 args + (self.h.data_ptr(), norm_w.data_ptr(), keep.data_ptr(), keep.shape[0],
                         out.data_ptr()))]

    def _norm_silu(self, h_ord, w_ord, lin):
        qw, layout, sc, qz = self._weight(lin, True)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        return self._with_geometry(("mtl_w4_gemm_norm_silu",
                (h_ord.data_ptr(), w_ord.data_ptr(), self.slots.data_ptr(),
                 ctypes.c_float(self.m.cfg.eps), lin.in_features, qw.data_ptr(), sc.data_ptr(),
                 p(qz), lin.out_features, lin.group_size, lin.zero_offset, layout,
                 self.act.data_ptr())), "gate_up")

    def _residual(self, x, xpart_name, lin, scatter, h_ord, name="down", halves=False):
        """``halves``: the partials hold [gate | up] (a bf16-kept up_proj beside its int4
        gate) instead of the 32-column gate|up interleave."""
        qw, layout, sc, qz = self._weight(lin, self.strip)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        xpart = self.part[xpart_name] if xpart_name else None
        xsplits = (self.splits[xpart_name] | (N.XPART_HALVES if halves else 0)) if xpart_name else 0
        return self._with_geometry(("mtl_w4_gemm_residual",
                (p(x), p(xpart), xsplits,
                 2 * lin.in_features if xpart_name else 0, lin.in_features, qw.data_ptr(),
                 sc.data_ptr(), p(qz), lin.out_features, lin.group_size,
                 lin.zero_offset, layout, self.h.data_ptr(), p(scatter), p(h_ord),
                 self.slots.data_ptr(), self.res_ws.data_ptr(), self.res_ws.numel())), name)

    def _norm_partials(self, h_ord, w_ord, lin, n, name, strip=None):
        qw, layout, sc, qz = self._weight(lin, self.strip_gemv[name] if strip is None else strip)
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        out = self.part[name]
        return self._with_geometry(("mtl_w4_gemm_norm_partials",
                (h_ord.data_ptr(), w_ord.data_ptr(), self.slots.data_ptr(),
                 ctypes.c_float(self.m.cfg.eps), lin.in_features, qw.data_ptr(), sc.data_ptr(),
                 p(qz), n, lin.group_size, lin.zero_offset, layout, out.data_ptr(),
                 out.numel() * 4)), name)

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
                                      self.pos.data_ptr(), self.attn.data_ptr(), None, cfg.n_heads,
                                      cfg.n_kv_heads, cfg.head_dim, cfg.max_seq, scale,
                                      self.attn_ws.data_ptr(), self.attn_ws.numel())),
            self._gemm(self.attn, lyr["o"], cfg.hidden, N.EPI_RESIDUAL, self.h, self.h),
            ("mtl_rmsnorm", (self.h.data_ptr(), lyr["post_attention_layernorm"].data_ptr(),
                             self.x.data_ptr(), 1, cfg.hidden, eps)),
            self._gemm(self.x, lyr["gate_up"], 2 * cfg.intermediate, N.EPI_SILU_MUL, None, self.act),
            # gate|up already emits the SiLU*up channels in the down input order
            self._gemm(self.act, lyr["down"], cfg.hidden, N.EPI_RESIDUAL, self.h, self.h,
                       no_perm=lyr["act_in_down_order"]),
        ]

    def _build_plan(self) -> None:
        cfg = self.m.cfg
        lib = N.load()
        embed = (self.ids.data_ptr(), self.table_ptrs.numel(), self.table_ptrs.data_ptr(),
                 self.vocabs.data_ptr(), cfg.hidden, self.h.data_ptr())
        self._embed = [("mtl_embed_sum", embed)]
        self._layer0_in = []
        if self.plan in ("fused", "strip"):
            # layer 0's RMSNorm statistics and act-order copy of h: formed by the embedding
            # sum in the step, by a residual add without partials when layer 0 runs alone
            p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
            into = (p(self.inv_perm_qkv[0]), self.x_qkv.data_ptr(), self.slots.data_ptr())
            self._embed = [("mtl_embed_sum_stats", embed + into)]
            self._layer0_in = [("mtl_residual_add", (None, 0, self.h.data_ptr()) + into +
                                (cfg.hidden,))]
            self._keep_launches = {}
            self._layers = [self._layer_plan_resid(li) for li in range(cfg.n_layers)]
        elif self.plan == "staged":
            self._layers = [self._layer_plan_staged(li) for li in range(cfg.n_layers)]
        elif self.plan == "partials":
            self._layers = [self._layer_plan_fused(li) for li in range(cfg.n_layers)]
        else:
            self._layers = [self._layer_plan(li) for li in range(cfg.n_layers)]
        self._final = self._final_plan()
        self._fns = {name: getattr(lib, name) for name in
                     ("mtl_rmsnorm", "mtl_w4_gemm_fused", "mtl_qk_norm_rope_kv",
                      "mtl_decode_attention", "mtl_embed_sum", "mtl_bf16_gemv_argmax",
                      "mtl_advance_position", "mtl_w4_gemm_partials",
                      "mtl_qk_norm_rope_kv_partials", "mtl_residual_rmsnorm", "mtl_residual_add",
                      "mtl_w4_gemm_norm_partials", "mtl_decode_attention_fused",
                      "mtl_bf16_gemv_argmax_norm", "mtl_bf16_gemv", "mtl_w4_gemm_residual",
                      "mtl_w4_gemm_norm_silu", "mtl_bf16_gemv_norm", "mtl_silu_mul_f32",
                      "mtl_w4_gemm_partials_geom", "mtl_w4_gemm_norm_partials_geom",
                      "mtl_w4_gemm_residual_geom", "mtl_w4_gemm_norm_silu_geom",
                      "mtl_w4_gemm_norm_partials_bf16", "mtl_embed_sum_stats",
                      "mtl_bf16_gemv_argmax_norm_advance")}

    def _final_norm_plan(self) -> list:
        """Fold the last layer's pending residual and write ``h_final = RMSNorm(h)``."""
        m, cfg = self.m, self.m.cfg
        eps = ctypes.c_float(cfg.eps)
        if self.plan in ("unfused", "fused", "strip"):   # h is complete
            return [("mtl_rmsnorm", (self.h.data_ptr(), m.final_norm.data_ptr(),
                                     self.h_final.data_ptr(), 1, cfg.hidden, eps))]
        return [("mtl_residual_rmsnorm", (self.part["down"].data_ptr(), self.splits["down"],
                                          self.h.data_ptr(), self.h.data_ptr(),
                                          m.final_norm.data_ptr(), self.h_final.data_ptr(),
                                          None, cfg.hidden, eps))]

    def _final_plan(self) -> list:
        """Final norm, head, greedy token into ``ids``, position + 1."""
        m, cfg = self.m, self.m.cfg
        eps = ctypes.c_float(cfg.eps)
        if self.plan in ("staged", "fused", "strip"):   # the head applies the final norm
            # the argmax's last launch also advances the position
            final = [] if self.plan != "staged" else [self._flush_staged()]
            return final + [("mtl_bf16_gemv_argmax_norm_advance", (
                self.h.data_ptr(), m.final_norm.data_ptr(), self.slots.data_ptr(), eps,
                m.head.data_ptr(), cfg.vocab, cfg.hidden, self.logits.data_ptr(),
                ctypes.c_void_p(self.ids.data_ptr()), ctypes.c_void_p(self.pos.data_ptr()),
                self.head_ws.data_ptr(), self.head_ws.numel()))]
        else:
            final = self._final_norm_plan() + [
                ("mtl_bf16_gemv_argmax", (self.h_final.data_ptr(), m.head.data_ptr(), cfg.vocab,
                                          cfg.hidden, self.logits.data_ptr(),
                                          ctypes.c_void_p(self.ids.data_ptr()),
                                          self.head_ws.data_ptr(), self.head_ws.numel()))]
        return final + [("mtl_advance_position", (ctypes.c_void_p(self.pos.data_ptr()),))]

    def _flush_staged(self):
        return ("mtl_residual_add", (self.part["down"].data_ptr(), self.splits["down"],
                                     self.h.data_ptr(), None, None, self.slots.data_ptr(),
                                     self.m.cfg.hidden))

    # position of each int4 GEMV launch inside a layer's plan
    _GEMV_AT = {"fused": {"qkv": 0, "o": 2, "gate_up": 3, "down": 4},
                "strip": {"qkv": 0, "o": 2, "gate_up": 3, "down": 4},
                "staged": {"qkv": 1, "o": 3, "gate_up": 5, "down": 6},
                "partials": {"qkv": 1, "o": 4, "gate_up": 6, "down": 7},
                "unfused": {"qkv": 1, "o": 4, "gate_up": 6, "down": 7}}

    def gemv_launch(self, li: int, name: str):
        """The (C function name, args) of one layer's int4 GEMV exactly as the step issues it."""
        shift = 0
        if self.v_keep[li] and name != "qkv":
            shift += self._keep_launches[(li, "v")] - 1                    # a separate bf16 v
        if self.up_keep[li] and name == "down":
            shift += self._keep_launches[(li, "up")] - 1                   # a separate bf16 up
        return self._layers[li][self._GEMV_AT[self.plan][name] + shift]

    def run_gemv(self, li: int, name: str) -> None:
        """Issue only that GEMV (timing; its inputs are whatever the buffers hold)."""
        self._run([self.gemv_launch(li, name)])

    def attention_launch(self, li: int):
        """The (C function name, args) of one layer's decode attention as the step issues it
        (the first launch of the layer whose name is an attention entry)."""
        for launch in self._layers[li]:
            if launch[0] in ("mtl_decode_attention_fused", "mtl_decode_attention"):
                return launch
        raise RuntimeError("this plan has no separate attention launch")

    def run_attention(self, li: int) -> None:
        """Issue only that layer's attention at the current position (timing: it rewrites
        the cache row of that position from whatever the q|k|v buffer holds)."""
        self._run([self.attention_launch(li)])

    def _run(self, plan) -> None:
        stream = torch.cuda.current_stream(self.dev).cuda_stream
        for name, args in plan:
            N.check(self._fns[name](*args, stream), name)

    # -- eager pieces -----------------------------------------------------------------
    def run_layer(self, li: int) -> None:
        """One decoder layer on ``self.h`` at position ``self.pos`` (writes KV).

        In the partials plans the layer's residual add of the down projection happens at the
        start of the next layer (or the final norm); :meth:`flush_residual` applies it.
        """
        self._run((self._layer0_in if li == 0 else []) + self._layers[li])

    def flush_residual(self) -> None:
        """Partials plans: fold the pending down-projection partials into ``self.h``
        (the fused and unfused plans leave nothing pending)."""
        if self.plan == "staged":
            self._run([self._flush_staged()])
        elif self.plan == "partials":
            cfg = self.m.cfg
            lyr0 = self.m.layers[0]
            self._run([("mtl_residual_rmsnorm", (self.part["down"].data_ptr(), self.splits["down"],
                                                 self.h.data_ptr(), self.h.data_ptr(),
                                                 lyr0["input_layernorm"].data_ptr(),
                                                 self.x.data_ptr(), None, cfg.hidden,
                                                 ctypes.c_float(cfg.eps)))])

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
        with _capturing(g):
            self.run_step()
        torch.cuda.synchronize(self.dev)
        self.ids.copy_(saved_ids)
        self.pos.copy_(saved_pos)
        self.graph = g

    def step(self, token: int | None = None, pos: int | None = None) -> torch.Tensor:
        """One replayed step; returns the (device) next-token buffer. ``token`` and ``pos``
        (host ints) replace the device-side ones; ``ValueError`` for a token outside the
        embedding or a position outside the KV cache."""
        if self.graph is None:
            raise RuntimeError("call capture() first")
        if token is not None:
            _check_ids([int(token)], self.id_limits)
            self.ids.fill_(int(token))
        if pos is not None:
            self.pos.fill_(_check_pos(pos, self.m.cfg.max_seq))
        self.graph.replay()
        return self.ids

    # -- prompt: every prompt row per launch ---------------------------------------------
    def _prefill_io(self, rows: int) -> dict:
        """Prompt-row buffers, grown on demand and kept for later prompts."""
        pf = getattr(self, "_pf", None)
        if pf is not None and pf["rows"] >= rows:
            return pf
        cfg, dev, bf = self.m.cfg, self.dev, torch.bfloat16
        z = lambda n, dt=bf: torch.zeros(rows, n, dtype=dt, device=dev)  # noqa: E731
        pf = {"rows": rows, "ids": z(self.table_ptrs.numel(), torch.int64), "h": z(cfg.hidden),
              "x": z(cfg.hidden), "x_nat": z(cfg.hidden), "qkv": z(cfg.qkv_out),
              "q": z(cfg.n_heads * cfg.head_dim), "attn": z(cfg.hidden),
              "act": z(cfg.intermediate),
              "gate": z(cfg.intermediate) if any(self.up_keep) else None}
        lib = N.load()
        # the split count follows each GEMM's shape (a q|k without its kept v has fewer
        # column tiles, so more splits): the largest of the layers' partial buffers
        shapes = {(lyr[name].in_features, lyr[name].out_features)
                  for lyr in self.m.layers for name in ("qkv", "o", "down")}
        nbytes = max(int(lib.mtl_w4_gemm_prefill_partials_bytes(rows, k, n)) for k, n in shapes)
        pf["part"] = torch.empty(max(nbytes, 16) // 4, dtype=torch.float32, device=dev)
        # the norms' output staged for the q|k|v and gate|up GEMMs: its 32-channel sums
        pf["xsum"] = torch.empty(rows, max(cfg.hidden // 32, 1), dtype=torch.float32,
                                 device=dev)
        self._pf = pf
        return pf

    def _prefill_gemm(self, x, rows: int, lin, epilogue: int, y, ldy: int, stream) -> None:
        """One prompt-length int4 GEMM on the strip copy of ``lin`` (mtl_w4_gemm_prefill,
        or mtl_w4_gemm_prefill_qsz for the reference's records)."""
        qw, layout = lin.stream_weight(True)
        sc, qz = lin.strip_meta()
        ws = ops.prefill_workspace(self.dev, rows, lin.in_features, lin.out_features)
        if layout == N.LAYOUT_STRIP_QSZ:
            N.check(N.load().mtl_w4_gemm_prefill_qsz(
                x.data_ptr(), rows, x.stride(0), lin.in_features, qw.data_ptr(), sc.data_ptr(),
                lin.out_features, lin.group_size, epilogue, N.OUT_BF16, y.data_ptr(), ldy,
                None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel() * 4,
                stream), "mtl_w4_gemm_prefill_qsz")
            return
        N.check(N.load().mtl_w4_gemm_prefill(
            x.data_ptr(), rows, x.stride(0), lin.in_features, qw.data_ptr(), sc.data_ptr(),
            qz.data_ptr(), lin.out_features, lin.group_size, lin.zero_offset, epilogue,
            N.OUT_BF16, y.data_ptr(), ldy, None if ws is None else ws.data_ptr(),
            0 if ws is None else ws.numel() * 4, stream), "mtl_w4_gemm_prefill")

    def _prefill_staged(self) -> bool:
        """Whether the prompt's norms stage x for the GEMMs (pair order and 32-channel sums,
        mtl_rmsnorm_gather_staged / mtl_w4_gemm_prefill_staged)."""
        return self.fuse_split_sums and self.stage_prefill_x and self.m.cfg.hidden % 32 == 0

    def _prefill_gemm_staged(self, x, xsum, rows: int, lin, epilogue: int, y, ldy: int,
                             stream) -> None:
        """One prompt-length int4 GEMM on staged x (mtl_w4_gemm_prefill_staged)."""
        qw, layout = lin.stream_weight(True)
        sc, qz = lin.strip_meta()
        qsz = layout == N.LAYOUT_STRIP_QSZ
        ws = ops.prefill_workspace(self.dev, rows, lin.in_features, lin.out_features)
        N.check(N.load().mtl_w4_gemm_prefill_staged(
            x.data_ptr(), xsum.data_ptr(), rows, x.stride(0), lin.in_features, qw.data_ptr(),
            sc.data_ptr(), None if qsz else qz.data_ptr(), lin.out_features, lin.group_size,
            0 if qsz else lin.zero_offset, N.META_QSZ if qsz else N.META_GPTQ, epilogue,
            N.OUT_BF16, y.data_ptr(), ldy, None if ws is None else ws.data_ptr(),
            0 if ws is None else ws.numel() * 4, stream), "mtl_w4_gemm_prefill_staged")

    def _prefill_partials(self, x, rows: int, lin, part: torch.Tensor, stream,
                          xsum: torch.Tensor | None = None) -> int:
        """The K-split partial sums of a prompt-length q|k|v, o or down GEMM into ``part``
        (mtl_w4_gemm_prefill_partials; ``xsum``: x staged); returns the split count for the
        launch that sums them (mtl_qk_norm_rope_kv_rows_partials,
        mtl_residual_rmsnorm_gather)."""
        lib = N.load()
        qw, layout = lin.stream_weight(True)
        sc, qz = lin.strip_meta()
        qsz = layout == N.LAYOUT_STRIP_QSZ
        K, Nc = lin.in_features, lin.out_features
        N.check(lib.mtl_w4_gemm_prefill_partials(
            x.data_ptr(), None if xsum is None else xsum.data_ptr(), rows, x.stride(0), K,
            qw.data_ptr(), sc.data_ptr(),
            None if qsz else qz.data_ptr(), Nc, lin.group_size, 0 if qsz else lin.zero_offset,
            N.META_QSZ if qsz else N.META_GPTQ, part.data_ptr(), part.numel() * 4, stream),
            "mtl_w4_gemm_prefill_partials")
        return int(lib.mtl_w4_gemm_prefill_partials_bytes(rows, K, Nc)) // (rows * Nc * 4)

    def _prefill_residual_norm(self, x_in, rows: int, lin, norm_w, gather, out, stream) -> None:
        """``h += x_in @ lin`` and ``out = RMSNorm(h)`` gathered by ``gather``: the GEMM's
        split partials, then the split sum, residual add and norm in one launch (the bits
        of the GEMM's residual launch followed by mtl_rmsnorm_gather), out staged for the
        next GEMM when the prompt stages x."""
        cfg, pf = self.m.cfg, self._pf
        h, part = pf["h"], pf["part"]
        if not self.fuse_split_sums:
            self._prefill_gemm(x_in, rows, lin, N.EPI_RESIDUAL, h, cfg.hidden, stream)
            N.check(N.load().mtl_rmsnorm_gather(
                h.data_ptr(), cfg.hidden, norm_w.data_ptr(),
                None if gather is None else gather.data_ptr(), out.data_ptr(), cfg.hidden,
                rows, cfg.hidden, ctypes.c_float(cfg.eps), stream), "mtl_rmsnorm_gather")
            return
        splits = self._prefill_partials(x_in, rows, lin, part, stream)
        N.check(N.load().mtl_residual_rmsnorm_gather(
            part.data_ptr(), splits, part.numel() * 4, h.data_ptr(), cfg.hidden,
            norm_w.data_ptr(),
            None if gather is None else gather.data_ptr(), out.data_ptr(), cfg.hidden,
            pf["xsum"].data_ptr() if self._prefill_staged() else None, rows, cfg.hidden,
            ctypes.c_float(cfg.eps), stream), "mtl_residual_rmsnorm_gather")

    def prefill_rows(self, ids: torch.Tensor, pos0: int = 0) -> torch.Tensor:
        """Every layer over the prompt rows ``ids`` (int64 ``[L, n_tables]``: one id per
        embedding table) at positions ``pos0 .. pos0 + L - 1``, writing their K/V into the
        cache: the reference's quantized prefill (moss_tts_lite/fast.py:210-270), each
        launch covering all L rows.  Returns the residual stream after the last layer,
        bf16 ``[L, hidden]`` (a view of an internal buffer)."""
        m, cfg = self.m, self.m.cfg
        _check_ids(ids, self.id_limits)
        ids = ids.to(device=self.dev, dtype=torch.int64).reshape(-1, self.table_ptrs.numel())
        rows = ids.shape[0]
        if rows < 1 or pos0 < 0 or pos0 + rows > cfg.max_seq:
            raise ValueError("prompt rows do not fit the KV cache")
        pf = self._prefill_io(rows)
        pf["ids"][:rows].copy_(ids)
        lib = N.load()
        st = torch.cuda.current_stream(self.dev).cuda_stream
        eps = ctypes.c_float(cfg.eps)
        scale = ctypes.c_float(attention_scale(cfg))
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        h, x, qkv, q, attn, act = (pf[k] for k in ("h", "x", "qkv", "q", "attn", "act"))
        H, Hkv, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        N.check(lib.mtl_embed_rows(pf["ids"].data_ptr(), rows, self.table_ptrs.numel(),
                                   self.table_ptrs.data_ptr(), self.vocabs.data_ptr(), cfg.hidden,
                                   h.data_ptr(), st), "mtl_embed_rows")
        n_layers = len(m.layers)
        staged = self._prefill_staged()
        xsum = pf["xsum"] if staged else None
        for li, lyr in enumerate(m.layers):
            lq = lyr["qkv"]
            if li == 0 and staged:   # later layers' input norms ride on the previous down GEMM
                N.check(lib.mtl_rmsnorm_gather_staged(
                    h.data_ptr(), cfg.hidden, lyr["input_layernorm"].data_ptr(), p(lq.perm),
                    x.data_ptr(), cfg.hidden, xsum.data_ptr(), rows, cfg.hidden, eps, st),
                    "mtl_rmsnorm_gather_staged")
            elif li == 0:
                N.check(lib.mtl_rmsnorm_gather(h.data_ptr(), cfg.hidden,
                                               lyr["input_layernorm"].data_ptr(),
                                               p(lq.perm), x.data_ptr(), cfg.hidden, rows,
                                               cfg.hidden, eps, st), "mtl_rmsnorm_gather")
            fuse_qkv = self.fuse_split_sums
            if fuse_qkv:
                splits = self._prefill_partials(x, rows, lq, pf["part"], st, xsum)
            else:
                self._prefill_gemm(x, rows, lq, N.EPI_NONE, qkv, cfg.qkv_out, st)
            if self.v_keep[li]:
                # the bf16-kept v_proj (gptq.py:689-693) reads x in its natural order
                N.check(lib.mtl_rmsnorm_gather(h.data_ptr(), cfg.hidden,
                                               lyr["input_layernorm"].data_ptr(), None,
                                               pf["x_nat"].data_ptr(), cfg.hidden, rows,
                                               cfg.hidden, eps, st), "mtl_rmsnorm_gather")
                qkv[:rows, lq.out_features:] = torch.nn.functional.linear(
                    pf["x_nat"][:rows], lyr["v_keep"])
            if fuse_qkv:   # the split sum rides on the q/k norm launch
                part = pf["part"]
                N.check(lib.mtl_qk_norm_rope_kv_rows_partials(
                    part.data_ptr(), splits, part.numel() * 4, lq.out_features,
                    qkv.data_ptr() if self.v_keep[li] else None, cfg.qkv_out, rows, pos0,
                    lyr["q_norm"].data_ptr(), lyr["k_norm"].data_ptr(), m.rope_cos.data_ptr(),
                    m.rope_sin.data_ptr(), q.data_ptr(), m.k_cache[li].data_ptr(),
                    m.v_cache[li].data_ptr(), H, Hkv, D, cfg.max_seq, eps, st),
                    "mtl_qk_norm_rope_kv_rows_partials")
            else:
                N.check(lib.mtl_qk_norm_rope_kv_rows(
                    qkv.data_ptr(), cfg.qkv_out, rows, pos0, lyr["q_norm"].data_ptr(),
                    lyr["k_norm"].data_ptr(), m.rope_cos.data_ptr(), m.rope_sin.data_ptr(),
                    q.data_ptr(), m.k_cache[li].data_ptr(), m.v_cache[li].data_ptr(), H, Hkv, D,
                    cfg.max_seq, eps, st), "mtl_qk_norm_rope_kv_rows")
            N.check(lib.mtl_prefill_attention(
                q.data_ptr(), m.k_cache[li].data_ptr(), m.v_cache[li].data_ptr(), rows, pos0,
                attn.data_ptr(), cfg.hidden, p(self.inv_perm_o[li]), H, Hkv, D, cfg.max_seq,
                scale, st), "mtl_prefill_attention")
            self._prefill_residual_norm(attn, rows, lyr["o"], lyr["post_attention_layernorm"],
                                        lyr["gate_up"].perm, x, st)
            if self.up_keep[li]:
                # int4 gate and the bf16-kept up_proj (gptq.py:689-693), then SiLU(gate) * up
                # in bf16 as the reference's MLP forms it (model.py:40-44)
                gate = pf["gate"]
                if staged:
                    self._prefill_gemm_staged(x, xsum, rows, lyr["gate_up"], N.EPI_NONE, gate,
                                              cfg.intermediate, st)
                else:
                    self._prefill_gemm(x, rows, lyr["gate_up"], N.EPI_NONE, gate,
                                       cfg.intermediate, st)
                x_up = x
                if lyr["gate_up"].perm is not None or staged:   # up reads natural order
                    x_up = pf["x_nat"]
                    N.check(lib.mtl_rmsnorm_gather(h.data_ptr(), cfg.hidden,
                                                   lyr["post_attention_layernorm"].data_ptr(),
                                                   None, x_up.data_ptr(), cfg.hidden, rows,
                                                   cfg.hidden, eps, st), "mtl_rmsnorm_gather")
                up = torch.nn.functional.linear(x_up[:rows], lyr["up_keep"])
                torch.mul(torch.nn.functional.silu(gate[:rows]), up, out=act[:rows])
            elif staged:
                self._prefill_gemm_staged(x, xsum, rows, lyr["gate_up"], N.EPI_SILU_MUL, act,
                                          cfg.intermediate, st)
            else:
                self._prefill_gemm(x, rows, lyr["gate_up"], N.EPI_SILU_MUL, act,
                                   cfg.intermediate, st)
            if li + 1 < n_layers:   # the residual add and the next layer's input norm
                nxt = m.layers[li + 1]
                self._prefill_residual_norm(act, rows, lyr["down"], nxt["input_layernorm"],
                                            nxt["qkv"].perm, x, st)
            else:
                self._prefill_gemm(act, rows, lyr["down"], N.EPI_RESIDUAL, h, cfg.hidden, st)
        return h[:rows]

    def _final_norm_row(self, h_row: torch.Tensor) -> None:
        """``h_final = RMSNorm(h_row)`` (fast.py:268)."""
        cfg = self.m.cfg
        N.check(N.load().mtl_rmsnorm(h_row.data_ptr(), self.m.final_norm.data_ptr(),
                                     self.h_final.data_ptr(), 1, cfg.hidden,
                                     ctypes.c_float(cfg.eps),
                                     torch.cuda.current_stream(self.dev).cuda_stream),
                "mtl_rmsnorm")

    # -- prompt + greedy loop ---------------------------------------------------------
    def prefill(self, token_ids: torch.Tensor) -> None:
        """Fill the KV cache with a prompt, all prompt tokens per launch
        (:meth:`prefill_rows`), then the final norm, head and greedy token of the last one.

        Leaves ``ids`` = greedy next token, ``logits`` its logits and ``pos`` = prompt length.
        """
        toks = token_ids.to(device=self.dev, dtype=torch.int64).reshape(-1)
        cfg = self.m.cfg
        if toks.numel() > cfg.max_seq:
            raise ValueError("prompt longer than the KV cache")
        self.m.reset_cache()
        h = self.prefill_rows(toks.reshape(-1, 1))
        self._final_norm_row(h[-1])
        st = torch.cuda.current_stream(self.dev).cuda_stream
        N.check(N.load().mtl_bf16_gemv_argmax(
            self.h_final.data_ptr(), self.m.head.data_ptr(), cfg.vocab, cfg.hidden,
            self.logits.data_ptr(), ctypes.c_void_p(self.ids.data_ptr()), self.head_ws.data_ptr(),
            self.head_ws.numel(), st), "mtl_bf16_gemv_argmax")
        self.pos.fill_(toks.numel())

    def prefill_stepwise(self, token_ids: torch.Tensor) -> None:
        """The same prompt as one decode step per token (eager); same end state."""
        _check_ids(token_ids, self.id_limits)
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


class FastMossDecoder(FastDecoder):
    """The MOSS-TTS decode step on the int4 backbone: 33-way summed embedding of one
    row of ids, the layers, final norm and the output heads -- text logits + 32 audio
    heads (pad code -inf), or in the audio2 variant the 2-way head + audio heads
    (moss_tts_lite/fast.py:123-194).  Mirrors ``FastMossTTS.capture()/step(row, pos,
    audio2)`` (fast.py:272-325): the host passes the position; one graph per variant
    serves every cache length.
    """

    def __init__(self, model: Int4Backbone, plan: str = "strip",
                 strip_geometry: dict | None = None):
        if model.cfg.n_vq < 1:
            raise ValueError("FastMossDecoder needs a MOSS-shaped backbone (cfg.n_vq > 0)")
        self.graphs: dict | None = None
        self.part_graphs: dict | None = None
        super().__init__(model, plan, strip_geometry=strip_geometry)

    def _alloc_io(self) -> None:
        m, cfg, dev = self.m, self.m.cfg, self.m.device
        bf = torch.bfloat16
        self.ids = torch.zeros(1 + cfg.n_vq, dtype=torch.int64, device=dev)   # ids_row
        self.table_ptrs = torch.tensor([m.embed_tokens.data_ptr()] +
                                       [t.data_ptr() for t in m.emb_ext], dtype=torch.int64,
                                       device=dev)
        self.id_limits = [cfg.text_embed_rows] + [cfg.audio_vocab] * cfg.n_vq
        self.vocabs = torch.tensor(self.id_limits, dtype=torch.int64, device=dev)
        self.lt = torch.zeros(cfg.vocab, dtype=bf, device=dev)
        self.la = torch.zeros(cfg.n_vq, cfg.audio_vocab, dtype=bf, device=dev)
        self.two = torch.zeros(2, dtype=bf, device=dev)
        self.logits = self.lt

    def _final_plan(self) -> list:
        return self._final_variant(audio2=False)

    def _heads_variant(self, audio2: bool) -> list:
        """The output heads on ``h_final``: text (or 2-way) logits and the audio logits."""
        m, cfg = self.m, self.m.cfg
        hf = self.h_final.data_ptr()
        audio = ("mtl_bf16_gemv", (hf, m.head_audio.data_ptr(), cfg.n_vq * cfg.audio_vocab,
                                   cfg.hidden, self.la.data_ptr(), cfg.audio_vocab,
                                   cfg.audio_pad_code))
        if audio2:
            first = ("mtl_bf16_gemv", (hf, m.head_2way.data_ptr(), 2, cfg.hidden,
                                       self.two.data_ptr(), 0, 0))
        else:
            first = ("mtl_bf16_gemv", (hf, m.head.data_ptr(), cfg.vocab, cfg.hidden,
                                       self.lt.data_ptr(), 0, 0))
        return [first, audio]

    def _final_variant(self, audio2: bool) -> list:
        return self._final_norm_plan() + self._heads_variant(audio2)

    def run_step(self, audio2: bool = False) -> None:
        """One whole step, eager, at the position in ``pos`` (not advanced)."""
        self._run(self._embed)
        for plan in self._layers:
            self._run(plan)
        self._run(self._final_variant(audio2))

    def capture(self) -> None:
        """Capture one whole-step graph per head variant (text, audio2)."""
        if self.graphs is not None:
            return
        saved_ids, saved_pos = self.ids.clone(), self.pos.clone()
        s = torch.cuda.Stream(self.dev)
        s.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(s):
            for audio2 in (False, True, False):
                self.run_step(audio2)
        torch.cuda.current_stream(self.dev).wait_stream(s)
        torch.cuda.synchronize(self.dev)
        self.graphs = {}
        for audio2 in (False, True):
            g = torch.cuda.CUDAGraph()
            with _capturing(g):
                self.run_step(audio2)
            self.graphs[audio2] = g
        torch.cuda.synchronize(self.dev)
        self.ids.copy_(saved_ids)
        self.pos.copy_(saved_pos)

    def capture_parts(self) -> None:
        """Capture the step in two parts, for callers that decide the head variant after
        the backbone has started: the backbone (embedding, layers, final norm into
        ``h_final``) and one graph per head variant on ``h_final``."""
        if getattr(self, "part_graphs", None) is not None:
            return
        self.capture()
        saved_ids, saved_pos = self.ids.clone(), self.pos.clone()
        self.part_graphs = {}
        backbone = self._embed + [op for plan in self._layers for op in plan] + \
            self._final_norm_plan()
        for key, plan in (("backbone", backbone), (False, self._heads_variant(False)),
                          (True, self._heads_variant(True))):
            g = torch.cuda.CUDAGraph()
            with _capturing(g):
                self._run(plan)
            self.part_graphs[key] = g
        torch.cuda.synchronize(self.dev)
        self.ids.copy_(saved_ids)
        self.pos.copy_(saved_pos)

    def replay_backbone(self, pos: int) -> None:
        """The backbone of one step for the ids row already in ``ids``, at ``pos``."""
        self.pos.fill_(_check_pos(pos, self.m.cfg.max_seq))
        self.part_graphs["backbone"].replay()

    def replay_heads(self, audio2: bool = False) -> None:
        """The output heads on ``h_final`` (text + audio, or 2-way + audio)."""
        self.part_graphs[bool(audio2)].replay()

    def step(self, row: torch.Tensor | None, pos: int, audio2: bool = False):
        """Replay one decode step for ``row`` ([1 + n_vq] ids) at cache position ``pos``.

        ``ValueError`` for a position outside the KV cache or, for a host ``row``, an id
        outside its table. A row already on the device is used as is: an id outside its
        table there sums a zero row into the embedding.

        Returns ``(lt, la, h_final, two)`` like ``FastMossTTS.step``: the text logits
        (stale in the audio2 variant), audio logits ``[n_vq, audio_vocab]``, the normed
        final hidden state and the 2-way logits (stale in the text variant).
        """
        if self.graphs is None:
            raise RuntimeError("call capture() first")
        pos = _check_pos(pos, self.m.cfg.max_seq)
        if row is not None:
            src = torch.as_tensor(row).reshape(-1)
            if src.device.type == "cpu":      # host rows are checked; device rows are not
                _check_ids(src, self.id_limits)  # read back (a sync per step)
            if src.data_ptr() != self.ids.data_ptr():
                self.ids.copy_(src)
        self.pos.fill_(pos)
        self.graphs[bool(audio2)].replay()
        return self.lt, self.la, self.h_final, self.two

    def prefill(self, rows: torch.Tensor) -> torch.Tensor:
        """Fill the KV cache with a prompt of ``rows`` ([L, 1 + n_vq] ids), every row per
        launch (:meth:`prefill_rows`, moss_tts_lite/fast.py:251-270); returns ``h_final``,
        the final-normed hidden state of the last row.  Leaves ``pos`` = L, the first free
        cache position (the warm-up steps of :meth:`capture` write there, and the first
        real step overwrites it)."""
        rows = rows.to(device=self.dev, dtype=torch.int64).reshape(-1, 1 + self.m.cfg.n_vq)
        if rows.shape[0] > self.m.cfg.max_seq:
            raise ValueError("prompt longer than the KV cache")
        self.m.reset_cache()
        h = self.prefill_rows(rows)
        self._final_norm_row(h[-1])
        self.pos.fill_(rows.shape[0])
        return self.h_final

    def prefill_stepwise(self, rows: torch.Tensor) -> torch.Tensor:
        """The same prompt as one eager step per row; returns ``h_final`` of the last row."""
        _check_ids(rows, self.id_limits)
        rows = rows.to(device=self.dev, dtype=torch.int64).reshape(-1, 1 + self.m.cfg.n_vq)
        if rows.shape[0] > self.m.cfg.max_seq:
            raise ValueError("prompt longer than the KV cache")
        self.m.reset_cache()
        for t in range(rows.shape[0]):
            self.ids.copy_(rows[t])
            self.pos.fill_(t)
            self._run(self._embed)
            for plan in self._layers:
                self._run(plan)
        self._run(self._final_norm_plan())
        self.pos.fill_(rows.shape[0])
        return self.h_final

    def generate(self, n_steps: int, use_graph: bool = True) -> torch.Tensor:
        raise NotImplementedError("MOSS sampling runs on the host per step; call step()")
