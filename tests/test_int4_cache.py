"""INT4 weight cache (qnn_int4_cache_*), host only.

The cache's bytes are checked against the oracle's QuantizeInt4 restatement
(oracle/qnn_oracle.cpp) and read back with the `safetensors` package; the
selection, shard plan, index and fingerprint against oracle/formats.py, whose
fingerprint is hashlib's SHA-256 and whose time stamp is pinned below to a
literal.
"""
import fcntl
import json
import os
import time

import numpy as np
import pytest

import oracle
from oracle import formats as of

ck = pytest.importorskip("quicknn_amd.checkpoint")
from quicknn_amd import hip  # noqa: E402


def bf16(x):
    """The BF16 bits torch writes for fp32 values (round to nearest even)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(
        np.uint16)


def save(path, tensors, bf16_names=()):
    """Writes a safetensors file with the `safetensors` package (BF16 through torch)."""
    torch = pytest.importorskip("torch")
    import safetensors.torch as stt

    out = {}
    for k, v in tensors.items():
        t = torch.from_numpy(np.ascontiguousarray(v))
        out[k] = t.to(torch.bfloat16) if k in bf16_names else t
    stt.save_file(out, path)


def moe_checkpoint(tmp_path, experts=3, hidden=64, inter=40, seed=0):
    rng = np.random.default_rng(seed)
    t, names = {}, []
    for e in range(experts):
        for proj, shape in (("gate_proj", (inter, hidden)), ("up_proj", (inter, hidden)),
                            ("down_proj", (hidden, inter))):
            n = f"model.layers.0.mlp.experts.{e}.{proj}.weight"
            t[n] = (rng.standard_normal(shape) * 0.02).astype(np.float32)
            names.append(n)
    t["model.layers.0.mlp.gate.weight"] = rng.standard_normal((experts, hidden)).astype(np.float32)
    t["model.layers.0.mlp.shared_expert.up_proj.weight"] = rng.standard_normal((inter, hidden)).astype(np.float32)
    t["model.layers.0.self_attn.q_proj.weight"] = rng.standard_normal((hidden, hidden)).astype(np.float32)
    t["model.norm.weight"] = np.ones(hidden, np.float32)
    p = os.path.join(tmp_path, "model.safetensors")
    save(p, t, bf16_names={n for n in names if "down" in n})
    return p, t


def source_entries(files: "ck.SafeTensorFiles"):
    return [(f.path, f.header_json) for f in files.files]


def quantized_reference(v: np.ndarray, is_bf16: bool) -> np.ndarray:
    return oracle.quantize_int4(bf16(v) if is_bf16 else v)


def test_time_stamp_literal(tmp_path):
    """The time stamp format yyyymmddhhnnsszzz, pinned to a literal."""
    p = os.path.join(tmp_path, "f")
    open(p, "wb").close()
    stamp = 1709214307.123  # 2024-02-29 13:45:07.123 UTC
    os.utime(p, ns=(int(stamp * 1e9), 1709214307_123_000_000))
    assert of.write_time_utc(p) == "20240229134507123"


def test_expert_cache_build_and_reuse(tmp_path):
    import safetensors.numpy as sn

    p, t = moe_checkpoint(tmp_path)
    calls = []
    with ck.SafeTensorFiles.Open(p) as src:
        fp = of.fingerprint(source_entries(src), of.CACHE_FORMAT)
        assert ck.LLMInt4Cache.SourceFingerprint(src) == fp
        cache_root = os.path.join(tmp_path, "cache")
        with ck.LLMInt4Cache(src, cache_root, progress=lambda d, n: calls.append((d, n))) as c:
            assert c.Directory == os.path.join(cache_root, f"{of.CACHE_FORMAT}-{fp}")
            assert calls == [(0, 1), (1, 1)]
            names = [x.name for x in src.Tensors() if of.selected(x.name, x.shape, 0)]
            assert len(names) == 9 and all(".mlp.experts." in n for n in names)
            (shard, members), = of.shard_plan(names, 0)
            assert shard == "experts-00001-of-00001.safetensors"
            raw = open(os.path.join(c.Directory, of.EXPERT_INDEX), "rb").read()
            index = json.loads(raw.decode("utf-8-sig"))
            assert index == {"metadata": {"format": of.CACHE_FORMAT, "source_fingerprint": fp},
                             "weight_map": {n: shard for n in members}}
            # The shard, read by the safetensors package, holds QuantizeInt4 of every matrix.
            loaded = sn.load_file(os.path.join(c.Directory, shard))
            assert list(loaded) == sorted(members) or set(loaded) == set(members)
            total = 0
            for n in members:
                want = quantized_reference(t[n], "down" in n)
                assert loaded[n].dtype == np.uint8 and np.array_equal(loaded[n], want), n
                blk = c.Weight(n, t[n].shape[0], t[n].shape[1])
                assert blk.dtype == hip.DT_U8 and blk.encoding == hip.WE_NATIVE
                assert blk.shape == want.shape and np.array_equal(blk.data.reshape(want.shape), want)
                total += want.nbytes
            assert c.MappedBytes() == total
            hdr = of.parse_safetensors(os.path.join(c.Directory, shard))
            assert hdr["metadata"] == {"format": of.CACHE_FORMAT, "source_fingerprint": fp}
            assert len(hdr["header"]) % 8 == 0
            with pytest.raises(hip.ESafeTensorError):
                c.Weight(members[0], 41, 64)
            with pytest.raises(hip.ESafeTensorError):
                c.Weight("model.layers.0.mlp.gate.weight", 3, 64)
            shard_mtime = os.stat(os.path.join(c.Directory, shard)).st_mtime_ns
        # Reopening finds the committed index: no rebuild, no progress calls.
        calls.clear()
        with ck.LLMInt4Cache(src, cache_root, progress=lambda d, n: calls.append((d, n))) as c2:
            assert calls == [] and os.stat(os.path.join(c2.Directory, shard)).st_mtime_ns == shard_mtime
    # A new write time of the source gives a new fingerprint and a new cache.
    os.utime(p, ns=(time.time_ns(), time.time_ns() + 5_000_000_000))
    with ck.SafeTensorFiles.Open(p) as src:
        fp2 = ck.LLMInt4Cache.SourceFingerprint(src)
        assert fp2 != fp and fp2 == of.fingerprint(source_entries(src), of.CACHE_FORMAT)


def test_dense_scope_selection_and_shards(tmp_path):
    rng = np.random.default_rng(3)
    t = {}
    for i in range(34):
        t[f"model.language_model.layers.{i}.mlp.up_proj.weight"] = rng.standard_normal((8, 40)).astype(np.float32)
    t["lm_head.weight"] = rng.standard_normal((16, 40)).astype(np.float32)
    t["model.language_model.layers.0.linear_attn.in_proj_a.weight"] = np.ones((4, 40), np.float32)
    t["model.language_model.layers.0.linear_attn.in_proj_b.weight"] = np.ones((4, 40), np.float32)
    t["model.language_model.norm.weight"] = np.ones(40, np.float32)
    t["model.language_model.layers.0.conv1d.bias"] = np.ones((3, 40), np.float32)
    t["model.visual.blocks.0.attn.qkv.weight"] = np.ones((4, 40), np.float32)
    p = os.path.join(tmp_path, "model.safetensors")
    save(p, t)
    with ck.SafeTensorFiles.Open(p) as src:
        names = [x.name for x in src.Tensors() if of.selected(x.name, x.shape, 1)]
        assert len(names) == 35 and "lm_head.weight" in names
        plan = of.shard_plan(names, 1)
        assert [s for s, _ in plan] == ["weights-00001-of-00002.safetensors", "weights-00002-of-00002.safetensors"]
        assert [len(m) for _, m in plan] == [32, 3]
        calls = []
        with ck.LLMInt4Cache(src, os.path.join(tmp_path, "c"), lambda d, n: calls.append((d, n)),
                             scope=ck.IQ_DENSE) as c:
            fp = of.fingerprint(source_entries(src), of.DENSE_CACHE_FORMAT)
            assert os.path.basename(c.Directory) == f"{of.DENSE_CACHE_FORMAT}-{fp}"
            assert calls == [(0, 2), (1, 2), (2, 2)]
            index = json.loads(open(os.path.join(c.Directory, of.DENSE_INDEX), encoding="utf-8-sig").read())
            assert index["weight_map"] == {n: s for s, m in plan for n in m}
            for s, members in plan:
                hdr = of.parse_safetensors(os.path.join(c.Directory, s))
                assert [x[0] for x in hdr["tensors"]] == members
            for n in names:
                want = oracle.quantize_int4(t[n])
                assert np.array_equal(c.Weight(n, *t[n].shape).data.reshape(want.shape), want)
            with pytest.raises(hip.ESafeTensorError):
                c.Weight("model.language_model.layers.0.linear_attn.in_proj_a.weight", 4, 40)


def test_index_validation_and_legacy_reuse(tmp_path):
    p, t = moe_checkpoint(tmp_path, experts=1)
    root = os.path.join(tmp_path, ".quicknn-cache")
    with ck.SafeTensorFiles.Open(p) as src:
        with ck.LLMInt4Cache(src, root) as c:
            d = c.Directory
        index_path = os.path.join(d, of.EXPERT_INDEX)
        good = open(index_path, "rb").read()

        def reopen_with(index_obj):
            with open(index_path, "w") as f:
                json.dump(index_obj, f)
            with pytest.raises(hip.ESafeTensorError):
                ck.LLMInt4Cache(src, root)

        idx = json.loads(good.decode("utf-8-sig"))
        stale = json.loads(json.dumps(idx))
        stale["metadata"]["source_fingerprint"] = "0" * 64
        reopen_with(stale)
        for bad_name in ("../x.safetensors", "a/b.safetensors", "c:x", "a\\b", ""):
            bad = json.loads(json.dumps(idx))
            bad["weight_map"][next(iter(bad["weight_map"]))] = bad_name
            reopen_with(bad)
        reopen_with({"metadata": idx["metadata"]})
        with open(index_path, "wb") as f:
            f.write(good)
        with ck.LLMInt4Cache(src, root) as c:
            assert c.Directory == d
        # A cache of the legacy format name, under the sibling .envision-cache, is reused as it stands.
        legacy_fp = of.fingerprint(source_entries(src), of.LEGACY_CACHE_FORMAT)
        legacy = os.path.join(tmp_path, ".envision-cache", f"{of.LEGACY_CACHE_FORMAT}-{legacy_fp}")
        os.makedirs(legacy)
        os.rename(os.path.join(d, of.EXPERT_INDEX), os.path.join(tmp_path, "moved.json"))
        import safetensors.numpy as sn

        shard = "experts-00001-of-00001.safetensors"
        data = sn.load_file(os.path.join(d, shard))
        sn.save_file(data, os.path.join(legacy, shard),
                     metadata={"format": of.LEGACY_CACHE_FORMAT, "source_fingerprint": legacy_fp})
        with open(os.path.join(legacy, of.EXPERT_INDEX), "w") as f:
            json.dump({"metadata": {"format": of.LEGACY_CACHE_FORMAT, "source_fingerprint": legacy_fp},
                       "weight_map": {n: shard for n in data}}, f)
        with ck.LLMInt4Cache(src, root) as c:
            assert c.Directory == legacy
            n = next(iter(data))
            assert np.array_equal(c.Weight(n, *t[n].shape).data.reshape(data[n].shape), data[n])
        # A legacy shard whose own metadata disagrees is refused.
        sn.save_file(data, os.path.join(legacy, shard), metadata={"format": of.CACHE_FORMAT,
                                                                    "source_fingerprint": legacy_fp})
        with pytest.raises(hip.ESafeTensorError):
            ck.LLMInt4Cache(src, root)


def test_builder_errors(tmp_path):
    p, t = moe_checkpoint(tmp_path, experts=1)
    with ck.SafeTensorFiles.Open(p) as src:
        with pytest.raises(hip.EArgumentException):
            ck.LLMInt4Cache(src, "")
        # Another builder holds build.lock: this one fails instead of publishing the same shards.
        fp = of.fingerprint(source_entries(src), of.CACHE_FORMAT)
        d = os.path.join(tmp_path, "locked", f"{of.CACHE_FORMAT}-{fp}")
        os.makedirs(d)
        with open(os.path.join(d, "build.lock"), "w") as lock:
            fcntl.flock(lock, fcntl.LOCK_EX | fcntl.LOCK_NB)
            with pytest.raises(hip.EInOutError):
                ck.LLMInt4Cache(src, os.path.join(tmp_path, "locked"))
        assert not os.path.exists(os.path.join(d, of.EXPERT_INDEX))
        # The source changes during the build: nothing is published.
        def touch(done, total):
            if done == 0:
                os.utime(p, ns=(time.time_ns(), time.time_ns() + 7_000_000_000))
        with pytest.raises(hip.EInvalidOp):
            ck.LLMInt4Cache(src, os.path.join(tmp_path, "moving"), progress=touch)
        moving = os.path.join(tmp_path, "moving")
        for sub in os.listdir(moving):
            left = os.listdir(os.path.join(moving, sub))
            assert of.EXPERT_INDEX not in left and not any(x.endswith(".part") for x in left)
    # No weights selected; a 3-D expert tensor; an F16 expert.
    for bad, err in (({"model.norm.weight": np.ones(8, np.float32)}, hip.EArgumentException),
                     ({"model.layers.0.mlp.experts.0.up_proj.weight": np.ones((2, 4, 32), np.float32)},
                      hip.EArgumentException),
                     ({"model.layers.0.mlp.experts.0.up_proj.weight": np.ones((4, 32), np.float16)},
                      hip.EArgumentException)):
        q = os.path.join(tmp_path, "bad.safetensors")
        save(q, bad)
        with ck.SafeTensorFiles.Open(q) as src, pytest.raises(err):
            ck.LLMInt4Cache(src, os.path.join(tmp_path, "badcache"))
