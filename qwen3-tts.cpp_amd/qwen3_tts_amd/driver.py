"""Host driver of the device frame loop: the control flow of
TTSTransformer::generate (src/tts_transformer.cpp:3007-3371) over the C ABI.

The arithmetic of the loop (talker step, code predictor, samplers, step
embedding) runs on the GPU; this module only assembles the prefill rows
(host glue in the reference too, src/tts_transformer.cpp:1030-1186), sizes
the KV cache, and replays frames in chunks, applying the per-frame callback
and the opt-in repetition-loop truncation after each chunk in frame order.
Frames computed past an EOS / abort / truncation point are discarded, so the
output equals the reference's frame-by-frame loop.
"""
import numpy as np


class GenerateError(RuntimeError):
    pass


def build_prefill(dev, cfg, text, speaker=None, language_id=2050, instruct=None):
    """build_prefill_graph (src/tts_transformer.cpp:1030-1186) in one device
    call (q3t_dev_build_prefill).  Returns (prefill [n][d], trailing [m][d],
    tts_pad [d])."""
    if len(text) < 4:
        raise GenerateError("Need at least 4 text tokens for prefill")
    return dev.build_prefill(text, speaker, language_id, instruct)


def _rep_loop(frames, state, n_cb):
    """Opt-in repetition-loop detector (src/tts_transformer.cpp:3225-3254).
    Returns the truncation length or None."""
    nf = len(frames)
    is_rep = False
    for back in range(1, 7):
        if is_rep or back >= nf:
            break
        a, b = frames[nf - 1], frames[nf - 1 - back]
        if int(np.sum(a == b)) >= 10:
            is_rep = True
    if is_rep:
        if state["run"] == 0:
            state["start"] = nf - 1
        state["run"] += 1
    else:
        state["run"] = 0
    if state["run"] >= 5:
        return state["start"]
    return None


def generate(dev, cfg, text, speaker=None, max_len=64, language_id=2050, repetition_penalty=1.05, temperature=0.9,
             top_k=50, instruct=None, eos_bias=0.0, target_frames=0, rep_loop_detect=False, on_frame=None, seed=0,
             chunk=32, prefill_rows=None):
    """Returns int32 codes [n_frames][n_codebooks].  `prefill_rows`, when
    given, is (prefill, trailing, tts_pad) and skips build_prefill."""
    if max_len <= 0:
        return np.zeros((0, cfg.n_codebooks), np.int32)
    if prefill_rows is None:
        prefill_rows = build_prefill(dev, cfg, text, speaker, language_id, instruct)
    prefill, trailing, pad = prefill_rows
    plen = prefill.shape[0]
    required = plen + max_len + 8
    cap = dev.lib.q3t_dev_kv_capacity(dev.h)
    if cap < required or cap > max(required * 2, 512):
        dev.kv_reserve(required)
    dev.prefill(prefill, 0, want_hidden=False)
    dev.frames_begin(trailing, pad, plen, max_len, repetition_penalty, temperature, top_k, eos_bias, target_frames,
                     seed)
    out = []
    rep_frames, rep_state = [], {"run": 0, "start": 0}
    produced = 0
    while produced < max_len:
        n = min(chunk, max_len - produced)
        codes, eos = dev.frames_run(n)
        stop = False
        for f in range(codes.shape[0]):
            frame = produced + f
            out.append(codes[f])
            if on_frame is not None and not on_frame(codes[f], cfg.n_codebooks, frame):
                stop = True
                break
            if rep_loop_detect:
                rep_frames.append(codes[f])
            cut = _rep_loop(rep_frames, rep_state, cfg.n_codebooks)
            if cut is not None:
                out = out[:cut]
                stop = True
                break
        produced += codes.shape[0]
        if stop or eos or codes.shape[0] < n:
            break
    if not out:
        return np.zeros((0, cfg.n_codebooks), np.int32)
    return np.stack(out).astype(np.int32)


def stream_audio(dev, voc, cfg, text, speaker=None, max_len=64, chunk_frames=25, context_frames=48, on_audio=None,
                 frame_chunk=1, **gen_kw):
    """generate() with the streaming vocoder after it, as the reference's
    StreamDecoderDriver (src/qwen3_tts.cpp:271-316, tail flush :615-633):
    once chunk_frames new frames exist, decode_window decodes them with
    context_frames of warm-up before them and hands the new samples to
    on_audio(samples) (returning False stops generation).  The vocoder reads
    the frame loop's device code rows in place (Device.frame_codes_ptr): no
    host copy of codes feeds it.  Returns (codes, audio, n_windows)."""
    state = {"emitted": 0, "windows": 0, "aborted": False}
    audio = []

    def deliver(samples):
        if samples.size == 0:
            return True
        audio.append(samples)
        state["windows"] += 1
        if on_audio is not None and not state["aborted"]:
            return bool(on_audio(samples))
        return True

    def on_frame(row, ncb, frame):
        n = frame + 1
        if state["aborted"] or n - state["emitted"] < chunk_frames:
            return not state["aborted"]
        s = voc.decode_window(None, state["emitted"], n, context_frames, n_frames=n, device_ptr=dev.frame_codes_ptr())
        state["emitted"] = n
        if not deliver(s):
            state["aborted"] = True
            return False
        return True

    codes = generate(dev, cfg, text, speaker, max_len=max_len, on_frame=on_frame, chunk=frame_chunk, **gen_kw)
    total = codes.shape[0]
    if total > state["emitted"] and not state["aborted"]:
        deliver(voc.decode_window(None, state["emitted"], total, context_frames, n_frames=total,
                                  device_ptr=dev.frame_codes_ptr()))
    out = np.concatenate(audio) if audio else np.zeros(0, np.float32)
    return codes, out, state["windows"]


def generate_streams(dev, cfg, streams, chunk=32, n_ctx=None, logits=None):
    """Batched form of generate() over independent utterances.

    `streams` is a list of dicts, one per utterance, each with `prefill_rows`
    ((prefill, trailing, tts_pad) as build_prefill returns them) and the
    generate() controls max_len, repetition_penalty, temperature, top_k,
    eos_bias, target_frames, seed.  Every stream's codes equal what
    generate() returns for it alone; all streams advance together, one
    device graph launch per frame.  Returns a list of [n_frames][16] arrays.
    `logits`, a list, receives after every streams_run call the streams'
    talker logits [n_streams][codec_vocab].
    """
    if not streams:
        return []
    need = max(s["prefill_rows"][0].shape[0] + s.get("max_len", 64) + 8 for s in streams)
    dev.streams_reserve(len(streams), max(need, n_ctx or 0))
    args = []
    for b, s in enumerate(streams):
        prefill, trailing, pad = s["prefill_rows"]
        dev.stream_prefill(b, prefill)
        args.append(dict(trailing=trailing, tts_pad=pad, n_past=prefill.shape[0], max_len=s.get("max_len", 64),
                         repetition_penalty=s.get("repetition_penalty", 1.05), eos_bias=s.get("eos_bias", 0.0),
                         target_frames=s.get("target_frames", 0), temperature=s.get("temperature", 0.9),
                         top_k=s.get("top_k", 50), seed=s.get("seed", 0)))
    dev.streams_begin(args)
    out = [[] for _ in streams]
    live = [a["max_len"] > 0 for a in args]
    produced = 0
    max_len = max(a["max_len"] for a in args)
    while produced < max_len and any(live):
        n = min(chunk, max_len - produced)
        codes, eos = dev.streams_run(n)
        if logits is not None:
            logits.append(np.stack([dev.stream_logits(b) for b in range(len(streams))]))
        for b in range(len(streams)):
            if codes[b].shape[0]:
                out[b].append(codes[b])
            if eos[b] or sum(c.shape[0] for c in out[b]) >= args[b]["max_len"]:
                live[b] = False
        produced += n
    return [np.concatenate(o).astype(np.int32) if o else np.zeros((0, cfg.n_codebooks), np.int32) for o in out]
