import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "soraku-tts_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


def load_golden(name: str):
    """A golden fixture plus the oracle shape and generate() kwargs it was made with."""
    from oracle.model import Shape

    f = np.load(os.path.join(GOLDEN, name + ".npz"))
    sh = [int(v) for v in f["shape"]]
    s = Shape(d_model=sh[0], n_layers=sh[1], n_q_heads=sh[2], n_kv_heads=sh[3], head_dim=sh[4],
              trunk_inter=sh[5], depth_mult=sh[6], n_codebooks=sh[7], codebook_size=sh[8],
              text_vocab=sh[9], n_language=sh[10],
              tie_audio_head=bool(int(f["tie_audio_head"])) if "tie_audio_head" in f.files else True)
    gen = {}
    for k in f.files:
        if k.startswith("gen_"):
            v = float(f[k])
            gen[k[4:]] = None if v == -1 else v
    for k in ("top_k", "top_k_q0", "max_new_frames", "min_new_frames", "seed"):
        if gen.get(k) is not None:
            gen[k] = int(gen[k])
    return f, s, gen


@pytest.fixture(scope="session")
def hip_device():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")
