"""bench.py's contract on the CPU: more than one GPU is refused with a message
and a non-zero status before any GPU work, and the per-kernel work formulas
the rooflines divide by add up to the whole forward's FLOPs."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("cname", ["c1", "c2", "c3", "c4", "c5"])
def test_kernel_flops_add_up_to_the_forward(cname):
    b = _bench()
    from edgebert_amd import synth
    spec = synth.CONFIGS[cname]
    cfg = spec.model
    _, _, lengths = synth.make_inputs(spec)
    per_layer = sum(b.kernel_work(cfg, lengths, spec.batch, k)[0]
                    for k in ("gemm_qkv", "gemm_out", "gemm_ffn_up", "gemm_ffn_down", "attention"))
    assert per_layer * cfg.num_hidden_layers == pytest.approx(b.forward_flops(cfg, lengths), rel=1e-12)


def test_embedding_bytes_count_position_rows_once():
    b = _bench()
    from edgebert_amd import synth
    cfg = synth.MINILM_L6
    H = cfg.hidden_size
    # 256 sequences of 128 tokens: a word row in and a row out per token, the
    # 128 position rows once; the same batch with one sequence 8 tokens longer
    # adds 8 tokens' rows and 8 more position rows.
    a = b.kernel_work(cfg, [128] * 256, 256, "embed")[0]
    c = b.kernel_work(cfg, [128] * 255 + [136], 256, "embed")[0]
    assert c - a == 8 * (8 + 2 * H * 4) + 8 * H * 4
    assert a < 256 * 128 * (8 + 3 * H * 4)            # not a position row per token
