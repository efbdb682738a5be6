import json
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, "tests", "golden")

# mla36m-v1 (config/mla36m-v1.json:1-25 of the reference) and tiny-test
# (config/tiny-test.json:1).
MLA36M = dict(vocab_size=16384, max_sequence_length=2048, n_layers=10, d_model=512, n_heads=8,
              head_dim_nope=48, head_dim_rope=16, head_dim_value=64, q_lora_rank=192,
              kv_lora_rank=128, d_ff=1360, norm_epsilon=1e-5, rope_theta=10000.0)
TINY = dict(vocab_size=264, max_sequence_length=64, n_layers=2, d_model=32, n_heads=2,
            head_dim_nope=12, head_dim_rope=4, head_dim_value=16, q_lora_rank=16,
            kv_lora_rank=8, d_ff=64, norm_epsilon=1e-5, rope_theta=10000.0)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def tiny_fixture():
    d = np.load(os.path.join(GOLDEN, "tiny_forward.npz"))
    return dict(params=d["params"], tokens=d["tokens"], logits=d["logits"],
                config=json.loads(str(d["config"])), parameter_count=int(d["parameter_count"]))


@pytest.fixture(scope="session")
def gpu():
    """The HIP product library on cuda:0; GPU tests fail (not skip) if it is absent."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import cpp_inference_train_engine_amd as mla
    mla.lib()
    return mla
