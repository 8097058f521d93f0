"""Host-side checks of libmmr.so that need no GPU: the C ABI's exports, config
parsing and validation, the MMRTW001 reader's error paths, the fp16 codec and
the seeded weight generator."""
from __future__ import annotations

import hashlib
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT, load_golden


def header_symbols() -> list[str]:
    text = (ROOT / "include" / "mmr.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmr_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(mmr):
    syms = header_symbols()
    assert len(syms) > 50
    lib = mmr.lib()
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(mmr.EXPORTED) == syms  # the binding covers the whole ABI
    out = subprocess.run(["nm", "-D", "--defined-only", str(mmr.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (mmr_[a-z0-9_]+)", out))
    assert set(syms) <= exported


def test_default_config_matches_reference(mmr):
    # test_minimind_config.cpp:13-21
    c = mmr.default_config()
    assert (c.hidden_size, c.num_hidden_layers, c.vocab_size, c.num_attention_heads) == (768, 8, 6400, 8)
    assert (c.num_key_value_heads, c.head_dim, c.intermediate_size, c.max_position_embeddings) == (4, 96, 2432, 32768)
    assert c.rms_norm_eps == pytest.approx(1e-6) and c.rope_theta == pytest.approx(1e6)
    assert (c.bos_token_id, c.eos_token_id, c.tie_word_embeddings) == (1, 2, 1)


def test_config_file_parsing(mmr, tmp_path):
    p = tmp_path / "minimind_runtime_config.txt"
    p.write_text("# comment\n hidden_size = 512 \nnum_attention_heads=8\nvocab_size=100\n"
                 "tie_word_embeddings=True\nrms_norm_eps=1e-5\n\n")
    c = mmr.load_config(p)
    assert c.hidden_size == 512 and c.head_dim == 64 and c.vocab_size == 100
    assert c.intermediate_size == 2432  # reference quirk: default kept from hidden 768
    assert c.tie_word_embeddings == 1
    assert c.rms_norm_eps == pytest.approx(1e-5) and c.rope_theta == pytest.approx(1e6)
    p.write_text("hidden_size 512\n")
    with pytest.raises(mmr.MmrError, match="invalid runtime config line"):
        mmr.load_config(p)
    with pytest.raises(mmr.MmrError, match="failed to open"):
        mmr.load_config(tmp_path / "missing.txt")


def test_config_validation_rejects(mmr, tmp_path):
    # test_minimind_config.cpp:23-26: kv heads not dividing q heads
    bad = mmr.make_config(num_key_value_heads=3)
    with pytest.raises(mmr.InvalidArgument, match="divisible"):
        mmr.write_synthetic_model(tmp_path / "x", bad, 0)


def numpy_normals(seed: int, first: int, count: int, std: float) -> np.ndarray:
    """Independent restatement of the generator: SplitMix64 draws, Box-Muller."""
    gamma = np.uint64(0x9E3779B97F4A7C15)
    idx = np.arange(first, first + count, dtype=np.uint64)
    pair = idx // np.uint64(2)

    def draw(n):
        with np.errstate(over="ignore"):
            z = np.uint64(seed) + n * gamma
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            z = z ^ (z >> np.uint64(31))
        return (z >> np.uint64(11)).astype(np.float64) * 2.0 ** -53

    u1 = draw(np.uint64(2) * pair + np.uint64(1))
    u2 = draw(np.uint64(2) * pair + np.uint64(2))
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    z = np.where(idx % np.uint64(2) == 0, r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2))
    return (std * z).astype(np.float32)


def test_generator_matches_independent_restatement(mmr):
    got = mmr.synthesize_normals(0, 1000, 4096, 0.02)
    ref = numpy_normals(0, 1000, 4096, 0.02)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-9)
    r16 = mmr.synthesize_normals(0, 1000, 4096, 0.02, round_fp16=True)
    np.testing.assert_array_equal(r16, got.astype(np.float16).astype(np.float32))
    big = mmr.synthesize_normals(5, 0, 200000, 1.0)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01
    ids = mmr.synthesize_prompt(1, 512, 6400)
    assert ids.min() >= 0 and ids.max() < 6400 and len(set(ids.tolist())) > 450


@pytest.mark.parametrize("case", ["mini", "cfg0"])
def test_synthetic_weights_file_matches_fixture(mmr, tmp_path, case):
    g = load_golden(case)
    mmr.write_synthetic_model(tmp_path, mmr.make_config(**g["config"]), g["seed"], g["std"], g["round_fp16"])
    h = hashlib.sha256((tmp_path / "weights.bin").read_bytes()).hexdigest()
    assert h == g["weights_sha256"]
    assert mmr.has_runtime_model(tmp_path)
    assert not mmr.has_runtime_model(tmp_path / "nowhere")


def _write_dir(mmr, tmp_path):
    g = load_golden("mini")
    mmr.write_synthetic_model(tmp_path, mmr.make_config(**g["config"]), g["seed"], g["std"], g["round_fp16"])
    return tmp_path / "weights.bin"


@pytest.mark.parametrize("corrupt, message", [
    ("magic", "unsupported runtime weight format"),
    ("truncate", "failed to read"),
    ("name", "expected tensor"),
])
def test_weights_reader_errors(mmr, tmp_path, corrupt, message):
    # runtime_loader.cpp:110-130 failure modes; the reader fails before any device work
    w = _write_dir(mmr, tmp_path)
    data = bytearray(w.read_bytes())
    if corrupt == "magic":
        data[:8] = b"MMRTW999"
    elif corrupt == "truncate":
        data = data[: len(data) // 2]
    else:
        off = 8 + 8
        data[off:off + 5] = b"xodel"
    w.write_bytes(bytes(data))
    with pytest.raises(mmr.MmrError, match=message):
        mmr.Model.load(tmp_path)


def test_fp16_codec_matches_numpy(mmr):
    rng = np.random.default_rng(4)
    v = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s for s in (0.02, 1.0, 3000.0)] +
                       [np.array([65504, 65520, 2 ** -24, 2 ** -25, 3 * 2 ** -25, 0.0, -0.0], np.float32)])
    np.testing.assert_array_equal(mmr.f32_to_f16(v), v.astype(np.float16).view(np.uint16))
    h = v.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(mmr.f16_to_f32(h), h.view(np.float16).astype(np.float32))


def test_cli_tools_reject_bad_flags_before_touching_a_device(tmp_path):
    # argument errors are reported before any model (or GPU) is set up
    bindir = ROOT / "minimind-orangepi_amd" / "bin"
    proc = subprocess.run([str(bindir / "bench_decode"), "--kv", "f64"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "--kv" in proc.stderr
    proc = subprocess.run([str(bindir / "check_prefill_consistency")], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 1 and "usage: check_prefill_consistency" in proc.stderr


def test_availability_probes_without_a_device(mmr):
    # this container has no GPU: the probes answer 0 instead of failing
    assert mmr.device_count() == 0 or mmr.custom_ops_available()
    if mmr.device_count() == 0:
        assert not mmr.cube_matvec_available() and not mmr.cube_matmul_available() and not mmr.custom_ops_available()


def test_op_argument_checks_need_no_device(mmr):
    # shape validation happens on the host before any launch
    with pytest.raises(mmr.InvalidArgument, match="multiple of 8"):
        mmr.check(mmr.lib().mmr_matvec_f16(1, 4, 12, 1, None, 1, None))
    with pytest.raises(mmr.InvalidArgument, match="head_dim"):
        mmr.check(mmr.lib().mmr_attention_from_cache(1, 1, 4, 8, 2, 80, 1, 1, 1 << 20, 0, None))
    assert mmr.matvec_argmax_workspace_size(6400, 768) > 0
    assert mmr.matvec_argmax_workspace_size(6400, 770) == 0
    assert mmr.attention_workspace_size(8, 2, 96, 64) == 2 * 64 * 4 * 98 * 4


@pytest.mark.parametrize("case", ["cfg3", "cfg0", "mini"])
def test_prefill_partial_buffer_covers_every_chunk_row_count(mmr, case):
    # The prefill GEMMs write split-K partials [splits][rows][N] into one
    # buffer sized when the state is made.  A chunk of r <= C rows can take
    # more K splits than a full chunk (the tiling aims at a block count), so
    # the buffer must hold the largest splits x r x N over every r, not r = C.
    cfg = mmr.make_config(**load_golden(case)["config"])
    H, D, Hq, Hkv, F = (cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads,
                        cfg.intermediate_size)
    shapes = [((Hq + 2 * Hkv) * D, H), (H, Hq * D), (2 * F, H), (H, F)]  # (N, K): QKV, O, gate_up, down
    for C in (512, 333, 100, 17, 1):
        have = mmr.prefill_partial_floats(cfg, C)
        need = {r: max(mmr.gemm_k_splits(r, n, k) * r * n for n, k in shapes) for r in range(1, C + 1)}
        worst = max(need, key=need.get)
        assert need[worst] <= have, (case, C, worst, need[worst], have)
        assert have == need[worst]  # tight: nothing beyond the largest chunk's need
        if case == "cfg3" and C == 512:
            # the case the buffer once missed: a shorter chunk needs more than a full one
            assert need[worst] > need[C] and worst < C
    assert mmr.prefill_partial_floats(cfg, 0) == 0


@pytest.mark.parametrize("head_dim,tile", [(96, 64), (64, 64), (128, 32)])
def test_decode_split_buckets(mmr, head_dim, tile):
    # The decode step replays one graph per attention split count, and the KV
    # backing reserved before a capture covers every context that count serves,
    # so the count may never fall as the context grows.  Buckets: 8, 12, then 16
    # (the O-projection prologue merges up to 16) up to 24 tiles; then one tile
    # per split rounded up to a multiple of 8, of 32 past 256 tiles, capped at
    # 512 (the attention kernels loop over the tiles past the cap).
    prev = 0
    for n_keys in range(1, 600 * tile, 7):
        s = mmr.decode_attention_splits(n_keys, head_dim)
        tiles = -(-n_keys // tile)
        assert s >= prev, (n_keys, s, prev)
        prev = s
        if tiles <= 8:
            assert s == 8
        elif tiles <= 12:
            assert s == 12
        elif tiles <= 24:
            assert s == 16
        elif tiles >= 512:
            assert s == 512
        else:
            step = 8 if tiles <= 256 else 32
            assert s % step == 0 and tiles <= s < tiles + step, (n_keys, tiles, s)
    assert mmr.decode_attention_splits(8193, 96) == 136  # 129 tiles of 64 keys
    for bad in ((0, 96), (100, 48), (100, 256)):
        with pytest.raises(mmr.InvalidArgument):
            mmr.decode_attention_splits(*bad)


def test_splitk_block_tiles_cover_the_grid_once(mmr):
    # Every (W row block, K chunk) of a batched split-K launch is computed by
    # exactly one block, whatever the grid; with the chunk count a multiple of
    # 8, the blocks of one chunk share an XCD (block b runs on XCD b mod 8).
    for row_blocks in (1, 3, 12, 18, 64, 100):
        for chunks in (1, 2, 3, 8, 12, 16, 24, 40):
            tiles = [mmr.splitk_block_tile(b, row_blocks, chunks) for b in range(row_blocks * chunks)]
            assert sorted(tiles) == [(r, c) for r in range(row_blocks) for c in range(chunks)], (row_blocks, chunks)
            if chunks % 8 == 0:
                xcd_of_chunk = {}
                for b, (_, c) in enumerate(tiles):
                    assert xcd_of_chunk.setdefault(c, b % 8) == b % 8, (row_blocks, chunks, c)
            else:
                assert tiles == [(b % row_blocks, b // row_blocks) for b in range(row_blocks * chunks)]
    with pytest.raises(mmr.MmrError):
        mmr.splitk_block_tile(12 * 16, 12, 16)
