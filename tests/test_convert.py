"""The checkpoint converter's host side (no GPU): the safetensors reader, the
bf16/fp16/fp32 -> fp16 conversion the reference's front end applies
(preprocess_layer_fixed_gpu.py:91-108, extract_*.py: torch .to(float32)
.to(float16)), the bucket-file writer's layout and the layer count.

Pins: the reader against the safetensors package's own numpy loader (F16 and
F32 tensors; its numpy backend has no bf16); the bf16 rounding against known
answers and against rounding the exact value from float64."""
import numpy as np
import pytest

from conftest import f32_to_bf16_bits, write_safetensors


def test_reader_matches_safetensors_package(conv, tmp_path):
    from safetensors.numpy import load_file
    rng = np.random.default_rng(0)
    a16 = rng.normal(0, 1, (24, 40)).astype(np.float16)
    a32 = rng.normal(0, 3, (7, 5)).astype(np.float32)
    p = str(tmp_path / "model.safetensors")
    write_safetensors(p, {"a16": ("F16", a16.shape, a16), "a32": ("F32", a32.shape, a32)})
    ref = load_file(p)
    st = conv.SafeTensors(str(tmp_path))
    assert st.names() == ["a16", "a32"]
    assert np.array_equal(st.fp16("a16").view(np.uint16), ref["a16"].view(np.uint16))
    assert np.array_equal(st.fp16("a32").view(np.uint16), ref["a32"].astype(np.float16).view(np.uint16))
    with pytest.raises(KeyError):
        st.fp16("missing")


def test_bf16_to_fp16_known_answers(conv, tmp_path):
    # bf16 bits -> expected fp16 bits
    cases = [
        (0x3F80, 0x3C00),   # 1.0
        (0xBF80, 0xBC00),   # -1.0
        (0x477F, 0x7BF8),   # 65280, representable
        (0x4780, 0x7C00),   # 65536 > fp16 max: +inf
        (0x3380, 0x0001),   # 2^-24, the smallest fp16 subnormal
        (0x3300, 0x0000),   # 2^-25: a tie, to even (zero)
        (0x3340, 0x0001),   # 1.5 * 2^-25 rounds up
        (0x0000, 0x0000),
        (0x8000, 0x8000),   # -0
        (0x7F80, 0x7C00),   # +inf
        (0x3DCD, 0x2E68),   # 0.10009765625 = 0x1.9ap-4, exact in fp16
    ]
    bits = np.array([c[0] for c in cases], np.uint16)
    want = np.array([c[1] for c in cases], np.uint16)
    write_safetensors(str(tmp_path / "model.safetensors"), {"w": ("BF16", bits.shape, bits)})
    got = conv.SafeTensors(str(tmp_path)).fp16("w").view(np.uint16)
    assert [hex(v) for v in got] == [hex(v) for v in want]
    nan = np.array([0x7FC0], np.uint16)
    write_safetensors(str(tmp_path / "model.safetensors"), {"w": ("BF16", nan.shape, nan)})
    assert np.isnan(conv.SafeTensors(str(tmp_path)).fp16("w")[0])


def test_bf16_to_fp16_matches_exact_rounding(conv, tmp_path):
    """Every bf16 value is exact in float64; rounding it straight to fp16
    must give the converter's fp16 (which goes through fp32)."""
    rng = np.random.default_rng(1)
    bits = np.concatenate([f32_to_bf16_bits(rng.normal(0, s, 4000).astype(np.float32))
                           for s in (1e-6, 1e-3, 0.02, 1.0, 3e4)])
    write_safetensors(str(tmp_path / "model.safetensors"), {"w": ("BF16", bits.shape, bits)})
    got = conv.SafeTensors(str(tmp_path)).fp16("w")
    sign = np.where(bits >> 15, -1.0, 1.0)
    e = ((bits >> 7) & 0xFF).astype(np.int64)
    m = (bits & 0x7F).astype(np.float64)
    exact = sign * np.where(e == 0, m / 128.0 * 2.0 ** -126, (1.0 + m / 128.0) * 2.0 ** (e - 127.0))
    with np.errstate(over="ignore"):
        want = exact.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_sharded_index_and_layer_count(conv, tmp_path):
    a = np.arange(32, dtype=np.float32).reshape(2, 16)
    write_safetensors(str(tmp_path / "s1.safetensors"), {"model.layers.0.input_layernorm.weight": ("F32", (16,), a[0])})
    write_safetensors(str(tmp_path / "s2.safetensors"), {"model.layers.1.input_layernorm.weight": ("F32", (16,), a[1])})
    import json
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": {"model.layers.0.input_layernorm.weight": "s1.safetensors",
                                                  "model.layers.1.input_layernorm.weight": "s2.safetensors"}}, f)
    st = conv.SafeTensors(str(tmp_path))
    assert np.array_equal(st.fp16("model.layers.1.input_layernorm.weight"), a[1].astype(np.float16))
    assert conv.layer_count(st, str(tmp_path)) == 2
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"num_hidden_layers": 32}, f)
    assert conv.layer_count(st, str(tmp_path)) == 32


def test_bucket_file_layout(conv, tmp_path):
    """Shapes and bytes as save_bucketmul_binary writes them
    (preprocess_layer_fixed_gpu.py:245-282), with the metadata keys
    binary_loader.hpp parses."""
    out_dim, in_dim = 64, 8
    R, C = in_dim * 16, out_dim // 16
    rng = np.random.default_rng(2)
    b = rng.integers(0, 65536, (R, C)).astype(np.uint16)
    s = rng.integers(0, 65536, (R, 4)).astype(np.uint16)
    p = rng.integers(0, 65536, in_dim).astype(np.uint16)
    base = str(tmp_path / "layer0_q_proj_bucketmul_fp16")
    conv.write_bucket_files(base, b, s, p, out_dim, in_dim)
    assert np.array_equal(np.fromfile(base + "_buckets.bin", "<u2"), b.ravel())
    assert np.array_equal(np.fromfile(base + "_stats.bin", "<u2"), s.ravel())
    assert np.array_equal(np.fromfile(base + "_probes.bin", "<u2"), p)
    meta = {}
    for line in open(base + "_meta.txt"):
        if line.strip() and not line.startswith("#"):
            k, v = line.split(":", 1)
            meta[k.strip()] = v.split()
    assert meta["buckets_shape"] == ["1", str(R), str(C)]
    assert meta["stats_shape"] == ["1", str(R), "4"]
    assert meta["probes_shape"] == ["1", str(in_dim)]
    assert (meta["in_dim"], meta["out_dim"], meta["bsize"]) == ([str(in_dim)], [str(out_dim)], ["16"])


def test_unknown_dtype_refused(conv, tmp_path):
    a = np.zeros(4, np.int32)
    write_safetensors(str(tmp_path / "model.safetensors"), {"i": ("I32", (4,), a)})
    with pytest.raises(ValueError):
        conv.SafeTensors(str(tmp_path)).fp16("i")
