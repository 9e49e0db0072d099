"""CPU checks of the GGUF reader that models::open's validation maps to
(sh_gguf_inspect: gguf/mod.rs:161-230 container, llama.rs:1038-1090 keys and
tensors). Valid images describe the right model; every malformed image is
refused with SH_ERR_FORMAT / SH_ERR_UNSUPPORTED before a byte of tensor data
is used. The same reader source is also built with AddressSanitizer and UBSan
and driven over the malformed cases, every truncation of a real header and
thousands of deterministic mutations: no sanitizer report may appear."""
import ctypes as C
import os
import shutil
import subprocess

import pytest

from gguf_writer import T, tiny_llama
from seeker_amd import _native as N
from seeker_amd import synth as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "seeker_amd", "csrc")


def inspect(data: bytes):
    buf = C.create_string_buffer(data, len(data))
    d = N.sh_model_dims()
    rc = N.lib().sh_gguf_inspect(buf, len(data), C.byref(d))
    return rc, d, N.lib().sh_last_error().decode()


def test_valid_tiny_image():
    rc, d, msg = inspect(tiny_llama().to_bytes())
    assert rc == N.SH_OK, msg
    assert (d.n_layer, d.n_embd, d.n_head, d.n_head_kv, d.head_dim, d.n_ff, d.n_vocab) == (1, 256, 4, 2, 64, 512, 64)


def test_synthetic_config_images():
    for shape in (S.TINY_TARGET, S.TINY_DRAFT):
        with S.GgufImage(shape, seed=0) as img:
            rc, d, msg = inspect(bytes(img.bytes()))
        assert rc == N.SH_OK, msg
        assert (d.n_layer, d.n_embd, d.n_ff, d.n_vocab) == (shape.n_layer, shape.n_embd, shape.n_ff, shape.n_vocab)
        assert abs(d.rope_freq_base - shape.rope_base) < 1e-3


@pytest.mark.parametrize("kw", [dict(wtype=12, etype=12, out_type=14, mix=1), dict(wtype=13, etype=14, out_type=14,
                                                                                  mix=1), dict(wtype=14, etype=13)],
                         ids=["q4km", "q5km_q6k_embd", "q6k_q5k_embd"])
def test_kquant_mix_images_accepted(kw):
    """K-quant mixes (Q4_K_M / Q5_K_M-style: attn_v and ffn_down of even layers
    and output in Q6_K; Q5_K / Q6_K token embeddings) are accepted."""
    import dataclasses
    shape = dataclasses.replace(S.LlamaShape(2, 512, 8, 4, 1024, 300, 512), **kw)
    with S.GgufImage(shape, seed=1) as img:
        rc, d, msg = inspect(bytes(img.bytes()))
    assert rc == N.SH_OK, msg
    assert (d.n_layer, d.n_embd, d.n_ff) == (2, 512, 1024)


def _malformed():
    """(name, image bytes, expected status) for each malformed case."""
    cases = []

    def add(name, mut, status=N.SH_ERR_FORMAT):
        img = tiny_llama()
        mut(img)
        cases.append((name, img.to_bytes(), status))

    # the advisor's case: an under-declared K/V/o/gate/up tensor must be refused,
    # not read past its end by the repack of d (or ff) columns
    for nm in ("attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down", "attn_q"):
        add(f"{nm} short rows", lambda im, nm=nm: setattr(im.tensor(f"blk.0.{nm}.weight"), "ne",
                                                          [im.tensor(f"blk.0.{nm}.weight").ne[0] // 2,
                                                           im.tensor(f"blk.0.{nm}.weight").ne[1]]))
    add("attn_k rows", lambda im: setattr(im.tensor("blk.0.attn_k.weight"), "ne", [256, 64]))
    add("3-d matrix", lambda im: setattr(im.tensor("blk.0.attn_q.weight"), "ne", [256, 256, 2]))
    add("matrix with ne[3]", lambda im: setattr(im.tensor("blk.0.attn_q.weight"), "ne", [256, 128, 1, 2]))
    add("row not whole blocks", lambda im: setattr(im.tensor("blk.0.ffn_down.weight"), "ne", [500, 256]))
    add("element count overflow", lambda im: setattr(im.tensor("blk.0.ffn_up.weight"), "ne",
                                                     [2**32, 2**32, 2**8]))
    add("offset past end", lambda im: setattr(im.tensor("blk.0.ffn_up.weight"), "off", 1 << 40))
    add("offset wraps", lambda im: setattr(im.tensor("blk.0.ffn_up.weight"), "off", 2**64 - 64))
    add("missing tensor", lambda im: im.tensors.remove(im.tensor("blk.0.ffn_down.weight")))
    add("norm not f32", lambda im: setattr(im.tensor("blk.0.attn_norm.weight"), "type", 1))
    add("norm wrong length", lambda im: setattr(im.tensor("blk.0.ffn_norm.weight"), "ne", [128]))
    add("token_embd vocab mismatch", lambda im: setattr(im.tensor("output.weight"), "ne", [256, 65]))
    add("unknown tensor type", lambda im: setattr(im.tensor("blk.0.attn_q.weight"), "type", 99),
        N.SH_ERR_UNSUPPORTED)
    add("head counts", lambda im: im.set_meta("llama.attention.head_count_kv", 4, 3))
    add("zero heads", lambda im: im.set_meta("llama.attention.head_count", 4, 0))
    add("missing block_count", lambda im: setattr(im, "meta", [m for m in im.meta if m[0] != "llama.block_count"]))
    add("more blocks than tensors", lambda im: im.set_meta("llama.block_count", 4, 2))
    add("bad alignment", lambda im: im.set_meta("general.alignment", 4, 48))
    add("bad version", lambda im: setattr(im, "version", 7))
    add("tensor count beyond table", lambda im: setattr(im, "n_tensors", 1000))
    add("kv count beyond metadata", lambda im: setattr(im, "n_kv", 50))
    add("architecture", lambda im: im.set_meta("general.architecture", 8, "gpt9"), N.SH_ERR_UNSUPPORTED)
    add("negative eps", lambda im: im.set_meta("llama.attention.layer_norm_rms_epsilon", 6, -1.0))
    add("attn_q/k types differ", lambda im: (setattr(im.tensor("blk.0.attn_k.weight"), "type", 12),
                                             setattr(im.tensor("blk.0.attn_k.weight"), "ne", [256, 128])),
        N.SH_ERR_UNSUPPORTED)
    # Q8_0 layers with one K-quant matrix: neither all K-quants (the multi-group
    # path) nor uniform layers (the fused path)
    add("Q8_0 layers with a Q6_K attn_v", lambda im: setattr(im.tensor("blk.0.attn_v.weight"), "type", 14),
        N.SH_ERR_UNSUPPORTED)
    add("extra metadata array", lambda im: im.set_meta("general.junk", 9, list(range(4))))
    return cases


MALFORMED = _malformed()


@pytest.mark.parametrize("name,data,status", [c for c in MALFORMED if c[0] != "extra metadata array"],
                         ids=[c[0] for c in MALFORMED if c[0] != "extra metadata array"])
def test_malformed_image_refused(name, data, status):
    rc, _, msg = inspect(data)
    assert rc == status, (rc, msg)
    assert msg


def test_metadata_array_skipped():
    img = tiny_llama()
    img.set_meta("tokenizer.ggml.token_type", 9, list(range(64)))
    rc, _, msg = inspect(img.to_bytes())
    assert rc == N.SH_OK, msg


def test_every_truncation_refused():
    data = tiny_llama().to_bytes()
    hdr = data.index(b"blk.0.ffn_down.weight") + 64  # the whole tensor table
    for n in list(range(0, hdr + 8)) + [len(data) - 1, len(data) - 32]:
        rc, _, _ = inspect(data[:n])
        assert rc == N.SH_ERR_FORMAT, n


@pytest.fixture(scope="module")
def asan_driver(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("asan") / "gguf_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-o", str(out), os.path.join(CSRC, "gguf.cpp"),
           os.path.join(ROOT, "tests", "native", "gguf_fuzz.cpp")]
    subprocess.run(cmd, check=True)
    return str(out)


def _run(drv, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([drv] + args, capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return r.stdout


def test_asan_malformed_cases(asan_driver, tmp_path):
    files = []
    for i, (name, data, _) in enumerate(MALFORMED):
        p = tmp_path / f"case{i}.gguf"
        p.write_bytes(data)
        files.append(str(p))
    out = _run(asan_driver, files).splitlines()
    assert len(out) == len(MALFORMED)


def test_asan_mutations(asan_driver, tmp_path):
    p = tmp_path / "tiny.gguf"
    p.write_bytes(tiny_llama(n_layer=2).to_bytes())
    hist = dict(tuple(map(int, ln.split())) for ln in _run(asan_driver, ["--mutate", "6000", "7", str(p)]).split("\n")
                if ln)
    assert hist[N.SH_ERR_FORMAT] > 300  # the mutations do reach the checks


def test_asan_synthetic_config_image(asan_driver, tmp_path):
    with S.GgufImage(S.TINY_DRAFT, seed=3) as img:
        p = tmp_path / "draft.gguf"
        p.write_bytes(bytes(img.bytes()))
    out = _run(asan_driver, [str(p)])
    assert out.startswith("0 ")
    _run(asan_driver, ["--mutate", "40", "11", str(p)])
