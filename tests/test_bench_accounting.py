"""bench.py's roofline accounting against the figures derived independently from the layer
shapes (bytes per active expert, algorithmic flops, expected active experts, path choice), so
that a slip in a formula shows here and not as a wrong fraction in the report."""

from __future__ import annotations

import pytest

import bench


def test_bytes_per_expert_30b():
    s = bench.S30B
    # W13: 2 * 768 * 2048 e4m3 bytes + 12 * 16 fp32 scales; W2: 2048 * 768 + 16 * 6 scales
    assert s.gate_up_expert_bytes() == 2 * 768 * 2048 + 4 * 12 * 16 == 3_146_496
    assert s.expert_bytes() == 3_146_496 + 2048 * 768 + 4 * 16 * 6 == 4_719_744


def test_bytes_per_expert_235b():
    s = bench.S235B
    assert s.expert_bytes() == 3 * 4096 * 1536 + 4 * (24 * 32 + 32 * 12) == 18_878_976


def test_gate_up_bytes_and_flops():
    s = bench.S30B
    # activations in (fp8 + scales) and the intermediate out, on top of the weights: at the 30B
    # shape (I = 768) the 16-row down GEMM quantises h, so gate_up writes bf16 h only
    for T in (32, 64):
        S = T * 8
        assert s.gate_up_bytes(10, T) == 10 * 3_146_496 + T * 2048 + 4 * T * 16 + 2 * S * 768
    # at the 235B shape (I = 1536 > 1024) gate_up quantises h itself up to 2 pairs per expert
    # (S = 256 <= 2 E): its bf16 h is written and read back once and the e4m3 codes and scales are
    # written; above, bf16 h only (a separate launch quantises it)
    b = bench.S235B
    S = 32 * 8
    assert b.gate_up_bytes(10, 32) == (10 * b.gate_up_expert_bytes() + 32 * 4096 + 4 * 32 * 32 + 2 * S * 1536
                                       + 2 * S * 1536 + S * 1536 + 4 * S * 12)
    S = 64 * 8
    assert b.gate_up_bytes(10, 64) == 10 * b.gate_up_expert_bytes() + 64 * 4096 + 4 * 64 * 32 + 2 * S * 1536
    assert s.gate_up_flops(4096) == 2 * 4096 * 8 * 1536 * 2048
    # the whole layer at a 4096-token chunk: 9,437,184 flop per pair + the router
    assert s.layer_flops(4096) == pytest.approx(4096 * 8 * 9_437_184 + 4096 * 2 * 2048 * 128)
    assert s.layer_flops(4096) == pytest.approx(3.114e11, rel=1e-3)


@pytest.mark.parametrize("T,expected", [(1, 8.0), (8, 51.6), (32, 111.8), (64, 125.9), (128, 128.0)])
def test_expected_active_experts(T, expected):
    assert bench.S30B.expected_active(T) == pytest.approx(expected, abs=0.05)


def test_prefill_path_matches_library_choice():
    """bench labels a configuration MFMA-bound exactly where the library runs the 128-row
    prefill GEMM (16-row tiles up to 8 pairs per expert, then 128-row at these shapes)."""
    for shape in (bench.S30B, bench.S235B):
        for T in (1, 64, 128, 256, 257, 1024, 4096):
            S = T * bench.K_TOP
            bm = 16 if S <= 8 * shape.E else 128
            assert shape.prefill_path(T) == (bm == 128), (shape.name, T)


def test_weight_rotation_defeats_the_last_level_cache():
    """With bench's 16 copies of the 30B experts, a copy is revisited only after at least twice
    the 256 MB last-level cache of other weights, at every batch size."""
    layer = bench.Layer.__new__(bench.Layer)
    layer.shape = bench.S30B
    layer.copies = [None] * 16
    for T in (1, 8, 64, 256, 4096):
        n = layer.n_rot(T)
        per_step = layer.shape.layer_bytes(layer.shape.expected_active(T), T)
        assert 2 <= n <= 16 and (n - 1) * per_step >= bench.LLC_BYTES, (T, n)


def test_bf16_bytes():
    """bf16 experts: 2 bytes per weight, no scales: gate_up streams 2 * 2I * H per active expert
    (6,291,456 B at the 30B shape) plus x in and bf16 h out; the layer adds W2 and the router."""
    s = bench.S30B
    assert s.bf16_gate_up_bytes(1, 1) == 2 * 2 * 768 * 2048 + 2 * 2048 + 2 * 8 * 768
    assert s.bf16_gate_up_bytes(126, 64) == 126 * 6_291_456 + 2 * 64 * 2048 + 2 * 512 * 768
    assert s.bf16_layer_bytes(126, 64) == 126 * 9_437_184 + 2 * 128 * 2048 + 4 * 64 * 2048


def test_prefill_gate_up_bytes():
    """On the 128-row path gate_up writes the e4m3 codes of h and one fp32 scale per 128 codes."""
    s = bench.S30B
    S = 4096 * 8
    assert s.gate_up_bytes(128, 4096) == 128 * 3_146_496 + 4096 * 2048 + 4 * 4096 * 16 + S * 768 + 4 * S * 6


@pytest.mark.parametrize("shape,T,bound", [(bench.S30B, 64, "hbm"), (bench.S30B, 256, "hbm"),
                                           (bench.S30B, 4096, "hbm"), (bench.S235B, 64, "hbm"),
                                           (bench.S235B, 2048, "hbm")])
def test_roofline_bound_follows_intensity(shape, T, bound):
    """The bound is chosen by the launch's flop per algorithmic byte against the 625 flop/B ridge
    (5 PFLOP/s over 8 TB/s), not by the tile path: the 256-token batch (~32 flop/B) and even the
    4096-token chunk (~470 flop/B, all 128 experts' weights streamed) sit below it."""
    n_active = shape.expected_active(T)
    r = bench.roofline_for(shape, T, {"gemm_gate_up": 0.1}, n_active)
    intensity = shape.gate_up_flops(T) / shape.gate_up_bytes(n_active, T)
    assert r["bound"] == bound and (intensity >= 625) == (bound == "mfma")
    assert r["frac"] == (r["mfma_frac"] if bound == "mfma" else r["hbm_frac"])
    # both fractions from the same duration
    assert r["hbm_frac"] == pytest.approx(shape.gate_up_bytes(n_active, T) / 1e-4 / 8e12, abs=1e-4)
    assert r["mfma_frac"] == pytest.approx(shape.gate_up_flops(T) / 1e-4 / 5e15, abs=1e-4)


def test_mfma_bound_above_the_ridge():
    """A hypothetical 64k-token chunk (~2000 flop/B) is MFMA-bound."""
    r = bench.roofline_for(bench.S30B, 65536, {"gemm_gate_up": 1.0}, 128)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s"
