"""Delay-pattern MOSS-TTS generation over :class:`FastMossDecoder`, with the sampling on the
device and the per-step host decision off the GPU's critical path.

Mirrors ``generate_fast`` (moss_tts_lite/fast.py:343-610): the same arguments, the same
delay-pattern state machine and watchdog, and the same random stream.  The reference
samples on the host side of each step: up to 1 + 1 + 31 ``int(tensor)`` reads per step
(the text token, audio channel 0 and every other sampled channel, fast.py:487-530), each a
device-to-host wait with the GPU idle behind it, plus ``torch.unique`` for the repetition
penalty.  Here:

- every sampled token stays on the device: the sampler writes the next step's id row and
  the history row directly (no host round trip for the row, fast.py:536-539);
- the random draws are the reference's: ``torch.multinomial(p, 1)`` draws
  ``q = exponential_(1)`` over ``p``'s shape from the same generator and returns
  ``argmax(p / q)``, which this module does without the host-side validity checks that
  make ``multinomial`` wait (the identity is checked on the device against
  ``torch.multinomial`` in the tests); every call has the reference's shape and order, so
  the generator advances identically.  top-k, top-p and softmax are the reference's own
  tensor ops (sampling.py:9-126), in its dtypes;
- the repetition penalty (sampling.py:37-66) uses per-codebook presence masks kept on the
  device instead of ``torch.unique`` of the history: the same elements get the same
  arithmetic;
- the host reads back two numbers per step (the text token and audio channel 0, which
  drive the state machine and the watchdog) and does so after the next step's backbone is
  queued, so the GPU computes while the host waits.  The host then queues the heads of the
  variant the decision selects (text or 2-way) and the next sampling stage.

``stats`` (optional dict) receives ``steps``, ``wall_s`` and ``host_wait_s`` (time the host
spent blocked on the per-step read).
"""
from __future__ import annotations

import dataclasses
import math
import time

import torch
import torch.nn.functional as F

# MOSS-TTS token ids (moss_tts_lite/model.py:9-24)
N_VQ = 32
AUDIO_PAD_CODE = 1024
PAD_TOKEN_ID = 151643
IM_END_TOKEN_ID = 151645
AUDIO_START_TOKEN_ID = 151652
AUDIO_END_TOKEN_ID = 151653
AUDIO_GEN_SLOT_TOKEN_ID = 151656
AUDIO_DELAY_SLOT_TOKEN_ID = 151662
_INT64_MAX = 9223372036854775807

# watchdog (fast.py:327-333)
_WD_LOW_ENERGY_CH0 = frozenset(
    (9, 60, 109, 123, 163, 209, 216, 365, 399, 402, 421, 580, 715, 734,
     774, 795, 827, 888, 890, 936, 971, 996, 1001))
_WD_SEGMENT_FLOOR = 640
_WD_SEGMENT_BACKSTOP_RUN = 32


@dataclasses.dataclass
class GenResult:
    """Result of :func:`generate_fast` (the fields of moss_tts_lite's GenResultWatchdog)."""

    text_ids: torch.Tensor
    audio_frames: torch.Tensor
    finished: bool
    n_steps: int
    watchdog_triggered: bool = False
    watchdog_reason: str = ""
    watchdog_stats: dict = dataclasses.field(default_factory=dict)


# ---------------------------------------------------------------------------- sampling
def filter_top_k(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Keep the top_k largest of each row, -inf elsewhere (sampling.py:9-17)."""
    k = min(int(top_k), logits.shape[-1])
    vals, idx = torch.topk(logits, k, dim=-1)
    return torch.full_like(logits, float("-inf")).scatter(-1, idx, vals)


def filter_top_p(logits: torch.Tensor, top_p: float) -> torch.Tensor:
    """Remove the tail past cumulative probability top_p, keeping the most likely token
    (sampling.py:103-115); in place, like the reference."""
    probs = F.softmax(logits, dim=-1)
    sp, si = torch.sort(probs, descending=True, dim=-1)
    remove = torch.cumsum(sp, dim=-1) > top_p
    remove[..., 1:] = remove[..., :-1].clone()
    remove[..., 0] = False
    drop = torch.zeros_like(logits, dtype=torch.bool).scatter_(-1, si, remove)
    return logits.masked_fill_(drop, float("-inf"))


def penalize(logits: torch.Tensor, seen: torch.Tensor, penalty: float) -> torch.Tensor:
    """The repetition penalty of sampling.py:37-66 over the tokens marked in ``seen``
    (bool [V], broadcast over rows): positive logits divided by the penalty, the others
    multiplied, in the logits' dtype."""
    hit = seen.expand_as(logits)
    out = torch.where(hit & (logits > 0), logits / penalty, logits)
    return torch.where(hit & ~(logits > 0), logits * penalty, out)


def sample_rows(logits: torch.Tensor, *, top_k=None, top_p=None, do_sample=True,
                seen: torch.Tensor | None = None, penalty: float = 1.0,
                generator: torch.Generator | None = None) -> torch.Tensor:
    """``sample_token`` (sampling.py:70-99) for logits [..., V] on the device: the next
    token of each row, with the reference's random draws and no host wait."""
    if seen is not None and penalty != 1.0:
        logits = penalize(logits, seen, penalty)
    if not do_sample:
        return torch.argmax(logits, dim=-1)
    shape = logits.shape
    x = logits.view(-1, shape[-1])
    if top_k is not None and top_k > 0:
        x = filter_top_k(x, top_k)
    if top_p is not None and top_p < 1.0:
        x = filter_top_p(x, top_p)
    probs = F.softmax(x, dim=-1)
    q = torch.empty_like(probs).exponential_(1, generator=generator)   # multinomial's draw
    return torch.argmax(probs / q, dim=-1).view(shape[:-1])


# ---------------------------------------------------------------------------- generation
def _set(x: torch.Tensor, col: int) -> None:
    """``x[..., col] = -inf`` as a device fill (an indexed assignment of a Python number
    stages the number on the host, which graph capture refuses)."""
    x[..., col:col + 1].fill_(float("-inf"))


@dataclasses.dataclass
class _State:
    """The delay-pattern state machine of fast.py:423-450 (host integers)."""

    al: int
    dl: int
    is_audio: bool
    is_stopping: bool = False
    wd_stop: bool = False
    wd_reason: str = ""
    wd_silent_run: int = 0
    wd_peak_segment: int = 0


class _Sampler:
    """Device buffers and the per-step sampling stage.  The ops are issued eagerly: the host
    runs a step ahead of the GPU, so their launch cost is hidden (capturing each stage shape
    as a graph measured no faster: 410 against 417 generated steps/s)."""

    def __init__(self, dec, max_steps: int, prompt: torch.Tensor, penalty: float):
        dev = dec.dev
        cfg = dec.m.cfg
        self.dec = dec
        self.lt_buf = torch.full((cfg.vocab,), float("-inf"), dtype=torch.bfloat16, device=dev)
        self.pre_exclude0 = torch.tensor([PAD_TOKEN_ID, AUDIO_GEN_SLOT_TOKEN_ID,
                                          AUDIO_DELAY_SLOT_TOKEN_ID, AUDIO_END_TOKEN_ID],
                                         device=dev)
        self.rows = torch.empty(max_steps, 1 + N_VQ, dtype=torch.int64, device=dev)
        self.decision = torch.empty(2, dtype=torch.int64, device=dev)
        self.host = torch.empty(2, dtype=torch.int64, pin_memory=True)
        self.done = torch.cuda.Event()
        self.penalty = penalty
        self.seen0 = self.seen_rest = None
        if penalty != 1.0:   # the history's codes: channel 0, and channels 1.. together
            v = cfg.audio_vocab
            self.seen0 = torch.zeros(v, dtype=torch.bool, device=dev)
            self.seen_rest = torch.zeros(v, dtype=torch.bool, device=dev)
            self.seen0[prompt[:, 1]] = True
            self.seen_rest[prompt[:, 2:].reshape(-1)] = True

    def stage(self, t: int, st: _State, forced_text: int, sampling_text: bool, smask: list,
              p: dict) -> None:
        """Queue step t's sampling: the next id row into ``dec.ids`` and ``rows[t]``, and the
        two numbers the host reads into the pinned buffer."""
        self._ops(t, st, forced_text, sampling_text, smask, p)
        self.rows[t].copy_(self.dec.ids)
        self.host.copy_(self.decision, non_blocking=True)
        self.done.record()

    def _ops(self, t: int, st: _State, forced_text: int, sampling_text: bool, smask: list,
             p: dict) -> None:
        dec = self.dec
        ids = dec.ids
        if sampling_text:
            if st.is_audio and not p["text_do_sample"]:
                two = dec.two / p["text_temperature"]
                if t == 0:
                    _set(two, 1)
                pick = torch.argmax(two)
                tok = torch.where(pick == 0, AUDIO_GEN_SLOT_TOKEN_ID, AUDIO_DELAY_SLOT_TOKEN_ID)
            elif st.is_audio:
                buf = self.lt_buf
                buf.fill_(float("-inf"))
                g, d = AUDIO_GEN_SLOT_TOKEN_ID, AUDIO_DELAY_SLOT_TOKEN_ID
                buf[g:g + 1].copy_(dec.two[0:1] / p["text_temperature"])
                buf[d:d + 1].copy_(dec.two[1:2] / p["text_temperature"])
                if t == 0:
                    _set(buf, d)
                tok = sample_rows(buf.view(1, -1), top_p=p["text_top_p"], top_k=p["text_top_k"],
                                  do_sample=True)[0]
            else:
                lt = dec.lt / p["text_temperature"]
                lt = lt.index_fill(0, self.pre_exclude0, float("-inf"))
                if t == 0:
                    _set(lt, AUDIO_DELAY_SLOT_TOKEN_ID)
                if t <= N_VQ:
                    _set(lt, IM_END_TOKEN_ID)
                tok = sample_rows(lt.view(1, -1), top_p=p["text_top_p"], top_k=p["text_top_k"],
                                  do_sample=p["text_do_sample"])[0]
            ids[0].copy_(tok)
        else:
            ids[0].fill_(forced_text)
        ids[1:].fill_(AUDIO_PAD_CODE)
        if any(smask):
            la = dec.la / p["audio_temperature"]
            kw = dict(top_p=p["audio_top_p"], top_k=p["audio_top_k"],
                      do_sample=p["audio_do_sample"], penalty=self.penalty)
            if smask[0]:
                ch0 = la[0].view(1, -1)
                _set(ch0, AUDIO_PAD_CODE)
                ids[1].copy_(sample_rows(ch0, seen=self.seen0, **kw)[0])
            rest = [j for j in range(1, N_VQ) if smask[j]]
            if rest:   # a contiguous run of channels (the delay pattern's window)
                j0, j1 = rest[0], rest[-1] + 1
                assert j1 - j0 == len(rest)
                rl = la[j0:j1].clone()
                _set(rl, AUDIO_PAD_CODE)
                ids[1 + j0:1 + j1].copy_(sample_rows(rl, seen=self.seen_rest, **kw))
        if self.seen0 is not None:            # scatter: no host-side step, so capturable
            self.seen0.scatter_(0, ids[1:2], True)
            self.seen_rest.scatter_(0, ids[2:], True)
        self.decision.copy_(ids[0:2])

    def read(self) -> tuple[int, int]:
        self.done.synchronize()
        return int(self.host[0]), int(self.host[1])


def _forced_text(st: _State) -> tuple[int, bool]:
    """The text token the state machine forces this step, and whether the text is sampled
    instead (fast.py:466-479)."""
    nxt = PAD_TOKEN_ID
    if st.wd_stop:
        if st.dl == _INT64_MAX or st.dl < N_VQ:
            nxt = AUDIO_DELAY_SLOT_TOKEN_ID
        else:
            nxt = AUDIO_END_TOKEN_ID
            st.is_audio = False
    elif not st.is_stopping and st.dl < N_VQ:
        nxt = AUDIO_DELAY_SLOT_TOKEN_ID
    elif not st.is_stopping and st.dl == N_VQ:
        nxt = AUDIO_END_TOKEN_ID
        st.is_audio = False
    return nxt, (not st.is_stopping) and (not st.wd_stop) and st.dl > N_VQ


@torch.inference_mode()
def generate_fast(dec, prompt: dict, max_new_tokens=4096, seed=1234, greedy=False,
                  text_temperature=1.5, text_top_p=1.0, text_top_k=50, audio_temperature=1.7,
                  audio_top_p=0.8, audio_top_k=25, audio_repetition_penalty=1.0,
                  stats: dict | None = None, watchdog: bool = True,
                  watchdog_silence_frames: int | None = None,
                  watchdog_max_segment_frames: int | None = None,
                  max_requested_pause_s: float | None = None) -> GenResult:
    """Delay-pattern generation (moss_tts_lite/fast.py:343-610) on a
    :class:`~moss_tts_lite_amd.fast.FastMossDecoder`.  ``prompt["input_ids"]``: int64
    [1, L, 1 + n_vq].  Same arguments, state machine, watchdog and random stream as the
    reference; the sampled tokens stay on the device (see the module docstring)."""
    cfg = dec.m.cfg
    if cfg.n_vq != N_VQ:
        raise ValueError(f"generate_fast needs {N_VQ} audio codebooks, the model has {cfg.n_vq}")
    input_ids = prompt["input_ids"]
    if input_ids.dim() != 3 or input_ids.shape[0] != 1 or input_ids.shape[-1] != N_VQ + 1:
        raise ValueError(f"expected prompt input_ids [1, L, {N_VQ + 1}], got {tuple(input_ids.shape)}")
    mask = prompt.get("attention_mask")
    if mask is not None:
        am = torch.as_tensor(mask)
        am = am.unsqueeze(0) if am.dim() == 1 else am
        if tuple(am.shape) != (1, input_ids.shape[1]):
            raise ValueError(f"bad attention_mask shape {tuple(am.shape)}")
        if not bool(am.all()):
            raise NotImplementedError("batch=1 generate_fast() requires an all-True prompt mask")
    seq_len = int(input_ids.shape[1])
    if seq_len + max_new_tokens > cfg.max_seq:
        raise ValueError(f"prompt {seq_len} + max_new_tokens {max_new_tokens} "
                         f"exceeds KV cache {cfg.max_seq}")
    if greedy:
        text_temperature = audio_temperature = 0
    text_do_sample = text_temperature > 0
    audio_do_sample = audio_temperature > 0
    p = dict(text_temperature=text_temperature if text_do_sample else 1,
             audio_temperature=audio_temperature if audio_do_sample else 1,
             text_do_sample=text_do_sample, audio_do_sample=audio_do_sample,
             text_top_p=text_top_p, text_top_k=text_top_k, audio_top_p=audio_top_p,
             audio_top_k=audio_top_k)
    torch.manual_seed(seed)

    rows = input_ids[0].to(device=dec.dev, dtype=torch.int64)
    col0 = rows[:, 0].cpu()
    continuation = int(col0[-1]) in (AUDIO_START_TOKEN_ID, AUDIO_GEN_SLOT_TOKEN_ID)
    hit = (col0 == AUDIO_START_TOKEN_ID).nonzero()
    start_idx = int(hit[-1]) if hit.numel() else -1
    st = _State(al=seq_len - start_idx if (continuation and start_idx != -1) else 0,
                dl=_INT64_MAX, is_audio=continuation and start_idx != -1)
    wd_floor = (watchdog_max_segment_frames if watchdog_max_segment_frames is not None
                else _WD_SEGMENT_FLOOR)
    wd_sil = watchdog_silence_frames if watchdog_silence_frames is not None else 64
    if max_requested_pause_s is not None and max_requested_pause_s > 0:
        wd_sil = max(wd_sil, math.ceil((max_requested_pause_s + 2.0) * 12.5))
    wd_stats: dict = {}

    dec.capture_parts()
    sampler = _Sampler(dec, max_new_tokens, rows, audio_repetition_penalty)
    t0 = time.perf_counter()
    wait = 0.0
    dec.prefill(rows)                       # the time_step 0 heads read the prompt's h_final
    dec.replay_heads(st.is_audio)
    text_steps: list = []
    n_steps = 0
    pos = seq_len
    for t in range(max_new_tokens):
        forced, sampling_text = _forced_text(st)
        smask = [(st.al > j) and (st.dl == _INT64_MAX or j > st.dl - 1) for j in range(N_VQ)]
        sampler.stage(t, st, forced, sampling_text, smask, p)
        if t + 1 < max_new_tokens:          # the next backbone runs while the host decides
            dec.replay_backbone(pos)
        w0 = time.perf_counter()
        next_text, ch0_val = sampler.read()
        wait += time.perf_counter() - w0
        if next_text == AUDIO_START_TOKEN_ID:
            st.is_audio = True
        if next_text == IM_END_TOKEN_ID:
            st.is_stopping = True
        # watchdog (fast.py:523-541)
        if watchdog and not st.wd_stop and st.is_audio and st.dl == _INT64_MAX:
            st.wd_silent_run = st.wd_silent_run + 1 if ch0_val in _WD_LOW_ENERGY_CH0 else 0
            seg_bound = max(wd_floor, 2 * st.wd_peak_segment)
            if st.wd_silent_run >= wd_sil:
                st.wd_stop, st.wd_reason = True, "silence"
            elif st.al > seg_bound and st.wd_silent_run >= _WD_SEGMENT_BACKSTOP_RUN:
                st.wd_stop, st.wd_reason = True, "max_segment"
            if st.wd_stop:
                wd_stats = {"reason": st.wd_reason, "step": n_steps + 1,
                            "segment_frames": st.al, "silent_run": st.wd_silent_run,
                            "peak_completed_segment": st.wd_peak_segment,
                            "silence_threshold_frames": wd_sil,
                            "segment_bound_frames": seg_bound,
                            "max_requested_pause_s": max_requested_pause_s}
        # delay-pattern counters (fast.py:543-552)
        if next_text in (AUDIO_START_TOKEN_ID, AUDIO_GEN_SLOT_TOKEN_ID, AUDIO_DELAY_SLOT_TOKEN_ID):
            st.al += 1
        if next_text == AUDIO_END_TOKEN_ID:
            st.wd_peak_segment = max(st.wd_peak_segment, st.al)
            st.wd_silent_run = 0
            st.al = 0
        if st.dl == _INT64_MAX and next_text == AUDIO_DELAY_SLOT_TOKEN_ID:
            st.dl = 0
        if st.dl != _INT64_MAX:
            st.dl += 1
        if st.dl > N_VQ:
            st.dl = _INT64_MAX
        text_steps.append(next_text)
        n_steps += 1
        if st.is_stopping or (st.wd_stop and next_text == AUDIO_END_TOKEN_ID):
            break
        if t + 1 < max_new_tokens:          # step t + 1's heads, on the backbone just run
            dec.replay_heads(st.is_audio)
        pos += 1
    torch.cuda.synchronize(dec.dev)
    if stats is not None:
        stats.update(steps=n_steps, wall_s=time.perf_counter() - t0, host_wait_s=wait)
    frames = sampler.rows[:n_steps, 1:].cpu()
    return GenResult(text_ids=torch.tensor(text_steps, dtype=torch.long), audio_frames=frames,
                     finished=bool(st.is_stopping) or bool(wd_stats), n_steps=n_steps,
                     watchdog_triggered=bool(wd_stats), watchdog_reason=st.wd_reason,
                     watchdog_stats=wd_stats)
