"""GGUF reader (lrs_gguf_*) and writer, on the CPU: the parser's contract
(GgufFile::parse, crates/gguf/src/parse.rs:64-126; tensor_data file.rs:47-75)
and the error cases the reference's parser rejects (bad magic, version != 3,
nested arrays, truncation, tensors out of bounds), plus a model file round
trip: every tensor and config key written is read back unchanged."""
import os
import struct

import numpy as np
import pytest

import modelgen


@pytest.fixture()
def gg(lrs):
    from llama_rs_amd import gguf

    return gguf


def test_round_trip_of_a_tiny_model_file(lrs, orc, gg, tmp_path):
    for cfg, w, arch in ((modelgen.TINY, modelgen.host_model(orc, modelgen.TINY, seed=2), "qwen2"),
                         (modelgen.HY_TINY, modelgen.hybrid_host_model(orc, modelgen.HY_TINY, seed=2),
                          "qwen35")):
        path = str(tmp_path / f"{arch}.gguf")
        modelgen.write_model_gguf(path, cfg, w)
        f = gg.GgufFile(path)
        assert f.version == 3
        assert f.str("general.architecture") == arch
        assert f.u32(f"{arch}.block_count") == cfg["n_layer"]
        assert f.u32(f"{arch}.attention.key_length") == cfg["head_dim"]
        assert f.f32(f"{arch}.attention.layer_norm_rms_epsilon") == np.float32(cfg["rms_eps"])
        assert f.array_len("tokenizer.ggml.tokens") == cfg["vocab"]
        assert f.n_tensors == len(w)
        t, dims, data = f.tensor("blk.0.ffn_down.weight")
        assert t == w["blk.0.ffn_down"][0] and dims == [cfg["n_ff"], cfg["n_embd"]]
        assert np.array_equal(data, w["blk.0.ffn_down"][1].view(np.uint8))
        t, dims, data = f.tensor("output_norm.weight")
        assert t == 0 and dims == [cfg["n_embd"]]
        assert np.array_equal(data.view(np.float32), w["output_norm"][1])
        if arch == "qwen35":
            assert f.u32("qwen35.ssm.group_count") == cfg["dn_k_heads"]
            t, dims, _ = f.tensor("blk.0.ssm_conv1d.weight")
            assert dims == [cfg["dn_conv"], modelgen.hy_conv_dim(cfg)]
        f.close()


def _mini(kv=b"", n_kv=0, tensors=b"", n_t=0, version=3, magic=b"GGUF", data=b""):
    head = magic + struct.pack("<IQQ", version, n_t, n_kv) + kv + tensors
    head += b"\0" * ((-len(head)) % 32)
    return head + data


def _s(x: str) -> bytes:
    return struct.pack("<Q", len(x)) + x.encode()


@pytest.mark.parametrize("case", ["magic", "version", "nested", "truncated", "bounds", "blocks"])
def test_parser_rejects_bad_files(lrs, gg, tmp_path, case):
    kv = _s("a") + struct.pack("<I", 4) + struct.pack("<I", 7)
    t_ok = _s("t") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 8, 0)
    if case == "magic":
        b = _mini(kv, 1, magic=b"GGUX")
    elif case == "version":
        b = _mini(kv, 1, version=2)
    elif case == "nested":
        b = _mini(_s("arr") + struct.pack("<IIQ", 9, 9, 1), 1)
    elif case == "truncated":
        b = _mini(kv, 1)[:20]
    elif case == "bounds":  # one Q8_0 block (34 B) declared, 10 B of data present
        b = _mini(kv, 1, t_ok, 1, data=b"\0" * 10)
    else:  # 33 elements of Q8_0: not a whole number of blocks
        bad = _s("t") + struct.pack("<I", 1) + struct.pack("<Q", 33) + struct.pack("<IQ", 8, 0)
        b = _mini(kv, 1, bad, 1, data=b"\0" * 68)
    path = str(tmp_path / "bad.gguf")
    open(path, "wb").write(b)
    if case in ("bounds", "blocks"):
        f = gg.GgufFile(path)  # the header parses; the tensor's bytes are rejected
        with pytest.raises(lrs.ModelError):
            f.tensor("t")
        f.close()
    else:
        with pytest.raises(lrs.ModelError):
            gg.GgufFile(path)


def test_alignment_and_metadata_types(lrs, gg, tmp_path):
    """general.alignment moves the data section (parse.rs:113-121); typed reads
    refuse the wrong value type."""
    q = np.arange(34, dtype=np.uint8)
    path = str(tmp_path / "a.gguf")
    gg.write_gguf(path, [("x.u", "u32", 5), ("x.f", "f32", 0.25), ("x.s", "str", "hi"),
                         ("x.a", "arr", ("i32", [1, 2, 3]))],
                  [("t0", 8, [32], q.tobytes()), ("t1", 8, [32], q[::-1].tobytes())], alignment=64)
    f = gg.GgufFile(path)
    assert f.u32("x.u") == 5 and f.f32("x.f") == 0.25 and f.str("x.s") == "hi"
    assert f.array_len("x.a") == 3
    with pytest.raises(lrs.ModelError):
        f.f32("x.s")
    assert np.array_equal(f.tensor("t1")[2], q[::-1])
    assert f.u32("general.alignment") == 64
    f.close()
    assert os.path.getsize(path) % 64 == 0
