"""Host-side pieces of bench.py at the tiny shape: the CPU baseline's
plumbing (item order, timing fields) and the traffic-summary reader."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402
from soraku_amd.config import TINY  # noqa: E402
from soraku_amd.synthetic import synthetic_weights, utterance  # noqa: E402


def test_cpu_baseline_runs_two_utterances():
    w = synthetic_weights(TINY, 0)
    items, us = [], []
    rng = np.random.default_rng(3)
    for i in range(2):
        text, prompt = utterance(TINY, i, n_text=5 + i, n_prompt=3)
        items.append((text, prompt, np.array([1], np.int64)))
        us.append(rng.random((8, TINY.n_codebooks)))
    cb = bench.cpu_baseline(TINY, w, items, us, temperature=0.9, n_frames=2, n_warm=1,
                            unit="utterance-frames/s")
    assert cb["unit"] == "utterance-frames/s" and cb["value"] > 0 and cb["cores"] >= 1
    assert "prefixes 9/5" in cb["sample"]


def test_measured_traffic_reads_the_committed_summaries():
    for key in bench.TRAFFIC_PROFILES:
        t, kv = bench.measured_traffic(key)
        if t is None:
            continue
        assert t > 1e8 and all(k > 0 for k in kv)


def test_prof_summary_names_and_frames():
    from soraku_amd.prof_summary import _frames, short_name

    n = "void sk::(anonymous namespace)::attn_o_kernel<2, 2048, 1, sk::WF32>(sk::GemvArgs, sk::AttnArgs)"
    assert short_name(n) == "attn_o_kernel<2, 2048, 1, sk::WF32>"
    names = ["gemm_nt_kernel<0>", "final_norm_kernel", "a", "b", "final_norm_kernel", "a", "b",
             "final_norm_kernel", "a"]
    assert _frames(names) == [(1, 4), (4, 7)]
