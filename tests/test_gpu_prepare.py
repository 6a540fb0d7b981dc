"""A quantised float model (idempotent_llm_amd.prepare on a small random
Qwen3) through the rocm runtime: calibrated scales instead of the random-init
generator's, the same bits as the integer oracle — prefill logits and greedy
generation, eager and graphed."""

import numpy as np
import pytest
import torch

from floatmodel import small_float_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def prepared(tmp_path_factory):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from idempotent_llm_amd import prepare as P
    model = small_float_model()
    calib = np.random.default_rng(5).integers(0, 1000, (4, 64), dtype=np.int64)
    d = str(tmp_path_factory.mktemp("prepared_gpu"))
    P.prepare(d, model, calib, device="cpu", model_id="test-small-qwen3")
    return d


def test_quantised_model_on_device_equals_oracle(prepared):
    from idempotent_llm_amd.hashchain import chain_hashes
    from idempotent_llm_amd.model import IntQwen3
    from oracle.model import IntQwen3Oracle
    print("[quantised small Qwen3: rocm vs oracle]", flush=True)
    ids = np.random.default_rng(9).integers(0, 1000, (1, 24), dtype=np.int64)
    orc = IntQwen3Oracle(prepared)
    want_logits = orc.forward(ids, np.arange(24, dtype=np.int64)[None])[0]
    te, le = orc.generate(ids, 16)
    m = IntQwen3(prepared, backend="rocm")
    got, _, _, _ = m.forward(torch.from_numpy(ids).cuda(),
                             torch.arange(24, device="cuda")[None], guard=True)
    assert np.array_equal(got.cpu().numpy(), want_logits)
    for use_graph in (False, True):
        tg, lg = m.generate(torch.from_numpy(ids).cuda(), 16, use_graph=use_graph)
        assert tg.cpu().numpy().tolist() == te.tolist(), use_graph
        assert chain_hashes(lg) == chain_hashes(le), use_graph
