"""Host-side logic of the frame loop driver (no GPU): the opt-in
repetition-loop truncation (src/tts_transformer.cpp:3225-3254), replayed the
way the driver applies it after each chunk, and the synthetic-weight specs
(tensor names/shapes/types of create_tensors, src/tts_transformer.cpp:379-668,
and the converter's dtype policy, scripts/convert_tts_to_gguf.py:249-324)."""
import numpy as np

from qwen3_tts_amd import config
from qwen3_tts_amd.driver import _rep_loop
from qwen3_tts_amd.synth import F16, F32, Q8_0, tensor_specs


def run_detector(frames):
    rep_frames, state = [], {"run": 0, "start": 0}
    for i, f in enumerate(frames):
        rep_frames.append(np.asarray(f))
        cut = _rep_loop(rep_frames, state, 16)
        if cut is not None:
            return i, cut
    return None, None


def test_rep_loop_truncates_at_run_start():
    rng = np.random.default_rng(0)
    frames = [rng.integers(0, 2048, 16) for _ in range(10)]
    loop = [rng.integers(0, 2048, 16) for _ in range(2)]
    seq = frames + [loop[i % 2] for i in range(12)]
    stop, cut = run_detector(seq)
    # frame 12 is the first repeat (period 2); five repeats in a row end at frame 16
    assert (stop, cut) == (16, 12)


def test_rep_loop_needs_ten_matching_codes():
    rng = np.random.default_rng(1)
    base = rng.integers(0, 2048, 16)
    seq = [rng.integers(0, 2048, 16) for _ in range(3)]
    for i in range(10):
        f = base.copy()
        f[: 7] = rng.integers(0, 2048, 7)         # only 9 codes match the previous frame
        seq.append(f)
    assert run_detector(seq) == (None, None)


def test_tensor_specs_follow_converter_policy():
    cfg = config.full_06b()
    specs = {n: (t, ne) for n, t, ne in tensor_specs(cfg, "q8_0")}
    assert specs["talker.blk.0.attn_q.weight"] == (Q8_0, (1024, 2048))
    assert specs["talker.blk.27.ffn_down.weight"] == (Q8_0, (3072, 1024))
    assert specs["talker.codec_head.weight"][0] == F16
    assert specs["code_pred.lm_head.14.weight"] == (F16, (1024, 2048))
    assert specs["talker.text_embd.weight"] == (F16, (2048, 151936))
    assert specs["talker.blk.3.attn_q_norm.weight"] == (F32, (128, 1))
    n_params = sum(ne[0] * ne[1] for _, ne in specs.values())
    assert abs(n_params - 905.7e6) / 905.7e6 < 0.01
    f16 = {n: t for n, t, _ in tensor_specs(cfg, "f16")}
    assert f16["talker.blk.0.ffn_gate.weight"] == F16


class _Shape:
    """Byte size of a tensor from its spec alone (no data generated)."""

    def __init__(self, ttype, ne):
        n = ne[0] * ne[1]
        self.nbytes = n * 34 // 32 if ttype == Q8_0 else n * (2 if ttype == F16 else 4)


def _frame_bytes():
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")
    spec = importlib.util.spec_from_file_location("q3t_bench", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.frame_bytes


def test_frame_bytes_follow_the_unit_figures():
    """The bench's algorithmic bytes against figures fixed independently of
    its formula: Q8_0 talker layers 15,728,640 params each at 34/32 bytes
    (467,927,040 B for 28), the F16 codec head and code-predictor heads
    (2 bytes a weight), the code-predictor layers read by 15 passes, and
    114,688 B of talker KV per position (28 layers x 8 heads x 128 x fp16 K+V)."""
    cfg = config.full_06b()
    w = {n: (t, ne, _Shape(t, ne)) for n, t, ne in tensor_specs(cfg, "q8_0")}
    fb = _frame_bytes()
    assert fb(cfg, w, 201) - fb(cfg, w, 200) == 114_688
    layer_params = 1024 * 4096 + 2048 * 1024 + 2 * 1024 * 3072 + 3072 * 1024
    assert layer_params == 15_728_640
    q8 = layer_params * 34 // 32
    norms_talker = 28 * (2 * 1024 + 2 * 128) * 4 + 1024 * 4
    norms_cp = 5 * (2 * 1024 + 2 * 128) * 4 + 1024 * 4
    weights = 28 * q8 + 3072 * 1024 * 2 + norms_talker + 15 * (5 * q8 + norms_cp) + 15 * 2048 * 1024 * 2
    kv_row = 114_688 // 28
    per_frame_kv = 114_688 * 101 + 5 * kv_row * sum(g + 2 for g in range(15)) + 17 * 1024 * 2
    assert fb(cfg, w, 100) == weights + per_frame_kv
    # the multi-stream form: weights once, KV per stream
    assert fb(cfg, w, [100, 100]) == weights + 2 * per_frame_kv


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says why,
    before touching any device."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
