"""lrs_model_load_gguf: a model read from a GGUF file (LlamaConfig::from_gguf
+ GpuRawWeights / GpuAuxWeights::from_gguf) gives the same logits, bit for
bit, as the same weights uploaded through the model entry points, for the
dense (qwen2, with q/k/v biases) and the hybrid (qwen35) architectures; and
matches the oracle."""
import numpy as np
import pytest

import modelgen

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(lrs):
    c = lrs.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("name", ["dense", "hybrid"])
def test_gguf_model_equals_uploaded_model(lrs, orc, ctx, tmp_path, name):
    from llama_rs_amd.gguf import load_gguf

    if name == "dense":
        cfg = modelgen.TINY
        w = modelgen.host_model(orc, cfg, seed=31)
        direct = modelgen.gpu_model(lrs, ctx, cfg, w)
        om = orc.Model(cfg, w, kv_f16=True, threads=8)
    else:
        cfg = modelgen.HY_TINY
        w = modelgen.hybrid_host_model(orc, cfg, seed=31)
        direct = modelgen.gpu_hybrid_model(lrs, ctx, cfg, w)
        om = orc.HybridModel(cfg, w, kv_f16=True, threads=8)
    path = str(tmp_path / f"{name}.gguf")
    modelgen.write_model_gguf(path, cfg, w)
    m = load_gguf(ctx, path)
    toks = [5, 9, 2, 400, 17, 3]
    for p, t in enumerate(toks):
        a = m.decode(t, p)
        b = direct.decode(t, p)
        o = om.forward([t])
        assert np.array_equal(a, b), p
        assert np.linalg.norm(a - o) / np.linalg.norm(o) < 1e-3
    assert len(m) == len(toks)
    m.close()
    direct.close()


def test_gguf_loader_errors(lrs, orc, ctx, tmp_path):
    from llama_rs_amd.gguf import load_gguf, model_kv, write_gguf

    cfg = modelgen.TINY
    path = str(tmp_path / "missing.gguf")
    write_gguf(path, model_kv(cfg, "qwen2"), [])  # no tensors
    with pytest.raises(lrs.ModelError):
        load_gguf(ctx, path)
    with pytest.raises(lrs.ModelError):
        load_gguf(ctx, str(tmp_path / "absent.gguf"))
