"""The reference's generation loop restated for the tests, driving a FastMossDecoder.

``sample_token`` follows moss_tts_lite/sampling.py:9-126 op for op (the reference's own
tests keep such ports inline, tests/test_core.py:119-183): top-k via ``torch.topk`` and an
index put, top-p via softmax / sort / cumsum, the repetition penalty over
``torch.unique`` of the history, and ``torch.multinomial`` for the draw.  ``generate``
follows ``generate_fast`` (moss_tts_lite/fast.py:343-610): the delay-pattern state
machine, the watchdog and the host reads, one step at a time through
``FastMossDecoder.step`` (the whole-step graphs), with every decision read back to the host
as the reference does.  The device generator (moss_tts_lite_amd.generate) must give the
same tokens for the same seed.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from moss_tts_lite_amd import generate as GEN

N_VQ = GEN.N_VQ
PAD, IM_END = GEN.PAD_TOKEN_ID, GEN.IM_END_TOKEN_ID
A_START, A_END = GEN.AUDIO_START_TOKEN_ID, GEN.AUDIO_END_TOKEN_ID
A_GEN, A_DELAY = GEN.AUDIO_GEN_SLOT_TOKEN_ID, GEN.AUDIO_DELAY_SLOT_TOKEN_ID
A_PAD = GEN.AUDIO_PAD_CODE
MAX = GEN._INT64_MAX


def apply_top_k(logits, top_k):
    b, v = logits.shape
    vals, idx = torch.topk(logits, min(top_k, v), dim=-1)
    out = torch.full_like(logits, float("-inf"))
    out[torch.arange(b, device=logits.device).unsqueeze(-1), idx] = vals
    return out


def apply_top_p(logits, top_p):
    probs = F.softmax(logits, dim=-1)
    sp, si = torch.sort(probs, descending=True, dim=-1)
    rm = torch.cumsum(sp, dim=-1) > top_p
    rm[..., 1:] = rm[..., :-1].clone()
    rm[..., 0] = False
    drop = torch.zeros_like(logits, dtype=torch.bool).scatter_(dim=-1, index=si, src=rm)
    logits[drop] = float("-inf")
    return logits


def apply_penalty(logits, prev, penalty):
    if penalty == 1.0 or prev is None:
        return logits
    uniq = torch.unique(prev.reshape(-1))
    tl = logits[:, uniq]
    pos = tl > 0
    tl[pos] /= penalty
    tl[~pos] *= penalty
    logits[:, uniq] = tl
    return logits


def sample_token(logits, prev_tokens=None, repetition_penalty=1.0, top_p=None, top_k=None,
                 do_sample=True):
    v = logits.size(-1)
    if prev_tokens is not None and repetition_penalty != 1.0:
        logits = apply_penalty(logits, prev_tokens, repetition_penalty)
    if not do_sample:
        return torch.argmax(logits, dim=-1)
    shape = logits.shape
    x = logits.view(-1, v)
    if top_k is not None and top_k > 0:
        x = apply_top_k(x, top_k)
    if top_p is not None and top_p < 1.0:
        x = apply_top_p(x, top_p)
    return torch.multinomial(F.softmax(x, dim=-1), num_samples=1).view(shape[:-1])


@torch.inference_mode()
def generate(dec, input_ids, max_new_tokens=64, seed=1234, greedy=False, text_temperature=1.5,
             text_top_p=1.0, text_top_k=50, audio_temperature=1.7, audio_top_p=0.8,
             audio_top_k=25, audio_repetition_penalty=1.0, watchdog=True,
             watchdog_silence_frames=None, watchdog_max_segment_frames=None):
    """Returns (text tokens, audio frames [n, 32], watchdog reason)."""
    device = dec.dev
    input_ids = input_ids.to(device=device, dtype=torch.long)
    seq_len = int(input_ids.shape[1])
    if greedy:
        text_temperature = audio_temperature = 0
    text_do_sample = text_temperature > 0
    text_temperature = text_temperature if text_do_sample else 1
    audio_do_sample = audio_temperature > 0
    audio_temperature = audio_temperature if audio_do_sample else 1
    torch.manual_seed(seed)
    col0 = input_ids[0, :, 0]
    cont = int(col0[-1]) in (A_START, A_GEN)
    hit = (col0 == A_START).nonzero()
    start_idx = int(hit[-1]) if hit.numel() else -1
    al = seq_len - start_idx if (cont and start_idx != -1) else 0
    is_audio = cont and start_idx != -1
    dl = MAX
    is_stopping = False
    pre_exclude_mask0 = torch.tensor([PAD, A_GEN, A_DELAY, A_END], device=device)
    generation_ids = input_ids.clone()
    lt_buf = torch.full((dec.m.cfg.vocab,), float("-inf"), dtype=torch.bfloat16, device=device)
    text_steps, audio_steps = [], []
    pos = seq_len
    wd_stop, wd_reason, wd_silent_run, wd_peak = False, "", 0, 0
    wd_floor = watchdog_max_segment_frames if watchdog_max_segment_frames is not None else 640
    wd_sil = watchdog_silence_frames if watchdog_silence_frames is not None else 64
    dec.capture_parts()
    for t in range(max_new_tokens):
        if t == 0:
            dec.prefill(input_ids[0])
            dec.replay_heads(is_audio)
            lt_step, la_step, two_step = dec.lt, dec.la, dec.two
        else:
            lt_step, la_step, _, two_step = dec.step(None, pos, audio2=is_audio)
            pos += 1
        next_text = PAD
        if wd_stop:
            if dl == MAX or dl < N_VQ:
                next_text = A_DELAY
            else:
                next_text, is_audio = A_END, False
        elif not is_stopping and dl < N_VQ:
            next_text = A_DELAY
        elif not is_stopping and dl == N_VQ:
            next_text, is_audio = A_END, False
        if (not is_stopping) and (not wd_stop) and dl > N_VQ:
            if is_audio and not text_do_sample:
                two = two_step / text_temperature
                if t == 0:
                    two[1] = float("-inf")
                next_text = A_GEN if int(torch.argmax(two)) == 0 else A_DELAY
            elif is_audio:
                lt_buf.fill_(float("-inf"))
                lt_buf[A_GEN] = two_step[0] / text_temperature
                lt_buf[A_DELAY] = two_step[1] / text_temperature
                if t == 0:
                    lt_buf[A_DELAY] = float("-inf")
                next_text = int(sample_token(lt_buf.view(1, -1), top_p=text_top_p,
                                             top_k=text_top_k, do_sample=True)[0])
            else:
                lt = (lt_step / text_temperature).index_fill(0, pre_exclude_mask0, float("-inf"))
                if t == 0:
                    lt[A_DELAY] = float("-inf")
                if t <= N_VQ:
                    lt[IM_END] = float("-inf")
                next_text = int(sample_token(lt.view(1, -1), top_p=text_top_p, top_k=text_top_k,
                                             do_sample=text_do_sample)[0])
        if next_text == A_START:
            is_audio = True
        if next_text == IM_END:
            is_stopping = True
        smask = [(al > j) and (dl == MAX or j > dl - 1) for j in range(N_VQ)]
        nxt_audio = torch.full((1, N_VQ), A_PAD, device=device, dtype=torch.long)
        if any(smask):
            audio_logit = la_step / audio_temperature
            if smask[0]:
                ch0 = audio_logit[0].view(1, -1)
                ch0[..., A_PAD] = float("-inf")
                nxt_audio[0, 0] = int(sample_token(ch0, prev_tokens=generation_ids[:, :, 1],
                                                   repetition_penalty=audio_repetition_penalty,
                                                   top_p=audio_top_p, top_k=audio_top_k,
                                                   do_sample=audio_do_sample)[0])
            rest = [j for j in range(1, N_VQ) if smask[j]]
            if rest:
                rl = audio_logit[rest]
                rl[..., A_PAD] = float("-inf")
                tok = sample_token(rl, prev_tokens=generation_ids[:, :, 2:],
                                   repetition_penalty=audio_repetition_penalty,
                                   top_p=audio_top_p, top_k=audio_top_k, do_sample=audio_do_sample)
                for k, j in enumerate(rest):
                    nxt_audio[0, j] = int(tok[k])
        ch0_val = int(nxt_audio[0, 0])
        if watchdog and not wd_stop and is_audio and dl == MAX:
            wd_silent_run = wd_silent_run + 1 if ch0_val in GEN._WD_LOW_ENERGY_CH0 else 0
            seg_bound = max(wd_floor, 2 * wd_peak)
            if wd_silent_run >= wd_sil:
                wd_stop, wd_reason = True, "silence"
            elif al > seg_bound and wd_silent_run >= 32:
                wd_stop, wd_reason = True, "max_segment"
        if next_text in (A_START, A_GEN, A_DELAY):
            al += 1
        if next_text == A_END:
            wd_peak, wd_silent_run, al = max(wd_peak, al), 0, 0
        if dl == MAX and next_text == A_DELAY:
            dl = 0
        if dl != MAX:
            dl += 1
        if dl > N_VQ:
            dl = MAX
        row = torch.cat([torch.full((1, 1), next_text, device=device, dtype=torch.long),
                         nxt_audio], dim=1)
        generation_ids = torch.cat([generation_ids, row[:, None, :]], dim=1)
        dec.ids.copy_(row[0])
        text_steps.append(next_text)
        audio_steps.append(nxt_audio[0].cpu())
        if is_stopping or (wd_stop and next_text == A_END):
            break
    return text_steps, torch.stack(audio_steps), wd_reason
