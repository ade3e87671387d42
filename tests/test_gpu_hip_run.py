"""pk_hip_run on the GPU: every op through .npy files against the C oracle,
and the invalid-launch probe (the reference's hip_run contract,
lib/Runtime/hip_run_main.cpp:17-27, 278-337)."""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

from polykernel_amd import build as pkbuild
from polykernel_amd import metrics as mt
from polykernel_amd import synth
from tests.helpers import int_bf16

pytestmark = pytest.mark.gpu


def cli(*args):
    assert pkbuild.CLI.exists(), "pk_hip_run not built"
    print("pk_hip_run", *args, flush=True)
    r = subprocess.run([str(pkbuild.CLI), *map(str, args)], capture_output=True, text=True, timeout=120)
    return r


def save_bf16(path, bits):
    np.save(path, np.ascontiguousarray(bits, dtype=np.uint16).view("V2"))
    return path


def load_bf16(path):
    return np.load(path).view(np.uint16)


def test_neg_probe_catches_invalid_launch(gpu):
    r = cli("neg")
    assert r.returncode == 1, r.stderr
    assert "PASS - invalid launch CAUGHT" in r.stderr
    assert "launch-config error" in r.stderr


def test_matmul_and_fused_ops_match_oracle(gpu, oracle, tmp_path):
    M, N, K = 130, 65, 127  # the reference's non-tile shape (tests/kernels/test_hip_run.py:319-322)
    a, b = int_bf16((M, K), 1), int_bf16((K, N), 2)
    bias = synth.normal_bf16((N,), 3, 0.5)
    r = synth.normal_bf16((M, N), 4)
    A, B, BIAS, R = (save_bf16(tmp_path / f"{n}.npy", v) for n, v in (("a", a), ("b", b), ("bias", bias), ("r", r)))
    assert cli("matmul", A, B, tmp_path / "c.npy").returncode == 0
    assert np.array_equal(load_bf16(tmp_path / "c.npy"), oracle.matmul(a, b))
    assert cli("fused_matmul_bias_gelu", A, B, BIAS, tmp_path / "g.npy").returncode == 0
    assert np.array_equal(load_bf16(tmp_path / "g.npy"), oracle.fused_matmul_bias_gelu(a, b, bias))
    assert cli("fused_matmul_bias_residual", A, B, BIAS, R, tmp_path / "y.npy").returncode == 0
    assert np.array_equal(load_bf16(tmp_path / "y.npy"), oracle.fused_matmul_bias_residual(a, b, bias, r))
    # contraction mismatch is an error, not a crash
    bad = cli("matmul", A, A, tmp_path / "bad.npy")
    assert bad.returncode == 1 and "mismatch" in bad.stderr


def test_rowwise_ops_match_oracle(gpu, oracle, tmp_path):
    x = synth.normal_bf16((33, 768), 5)
    r = synth.normal_bf16((33, 768), 6)
    g = synth.normal_bf16((768,), 7, 0.1, 1.0)
    X, R, G = (save_bf16(tmp_path / f"{n}.npy", v) for n, v in (("x", x), ("r", r), ("g", g)))
    assert cli("rmsnorm", X, tmp_path / "n.npy", "--weight", G, "--epsilon", "1e-6").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "n.npy"), oracle.rmsnorm(x, g, 1e-6))
    assert cli("rmsnorm", X, tmp_path / "n0.npy").returncode == 0  # default eps 1e-5, no weight
    mt.assert_correct(load_bf16(tmp_path / "n0.npy"), oracle.rmsnorm(x, None, 1e-5))
    assert cli("fused_residual_rmsnorm", X, R, tmp_path / "rr.npy", "--weight", G, "--epsilon", "1e-6").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "rr.npy"), oracle.residual_rmsnorm(x, r, g, 1e-6))
    assert cli("softmax", X, tmp_path / "s.npy", "--axis", "-1").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "s.npy"), oracle.softmax(x))
    assert cli("softmax", X, tmp_path / "s.npy", "--axis", "0").returncode == 1
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert cli("gelu", save_bf16(tmp_path / "codes.npy", codes), tmp_path / "ge.npy").returncode == 0
    assert np.array_equal(load_bf16(tmp_path / "ge.npy"), oracle.gelu(codes))  # all 65536 codes
    lg = synth.normal_f32((17, 1000), 8, 2.0)
    mk = synth.mask_bf16((17, 1000), 9, 0.1)
    np.save(tmp_path / "lg.npy", lg)
    assert cli("fused_softmax_mask", tmp_path / "lg.npy", save_bf16(tmp_path / "mk.npy", mk),
               tmp_path / "sm.npy").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "sm.npy"), oracle.softmax_mask(lg, mk))
    assert cli("fused_rmsnorm_matmul", X, save_bf16(tmp_path / "w.npy", synth.normal_bf16((768, 256), 10, 0.036)),
               tmp_path / "rm.npy", "--epsilon", "1e-6", "--weight", G).returncode == 0
    w = load_bf16(tmp_path / "w.npy")
    rep = mt.report(load_bf16(tmp_path / "rm.npy"), oracle.fused_rmsnorm_matmul(x, w, g, 1e-6))
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99, rep


def test_quantize_and_int8_match_oracle(gpu, oracle, tmp_path):
    w = synth.normal_bf16((256, 96), 11, 0.06)
    a = synth.normal_bf16((5, 256), 12)
    W, A = save_bf16(tmp_path / "w.npy", w), save_bf16(tmp_path / "a.npy", a)
    assert cli("quantize", W, tmp_path / "wq.npy", tmp_path / "s.npy").returncode == 0
    wq, s = np.load(tmp_path / "wq.npy"), np.load(tmp_path / "s.npy")
    owq, os_ = oracle.quantize_per_channel(w)
    assert wq.dtype == np.int8 and np.array_equal(wq, owq) and np.array_equal(s, os_)  # bit-exact
    assert cli("matmul_int8", A, tmp_path / "wq.npy", tmp_path / "s.npy", tmp_path / "c.npy").returncode == 0
    rep = mt.report(load_bf16(tmp_path / "c.npy"), oracle.matmul_int8(a, owq, os_))
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99, rep


def test_attention_and_kv_ops_match_oracle(gpu, oracle, tmp_path):
    B, H, Sc, Sq, D = 1, 2, 64, 32, 64
    q = synth.normal_bf16((B, H, Sq, D), 13)
    kc = synth.normal_bf16((B, H, Sc, D), 14)
    vc = synth.normal_bf16((B, H, Sc, D), 15)
    kn = synth.normal_bf16((B, H, Sq, D), 16)
    vn = synth.normal_bf16((B, H, Sq, D), 17)
    Q, KC, VC, KN, VN = (save_bf16(tmp_path / f"{n}.npy", v)
                         for n, v in (("q", q), ("kc", kc), ("vc", vc), ("kn", kn), ("vn", vn)))
    assert cli("kv_cache_update", KC, KN, tmp_path / "k.npy").returncode == 0
    k = load_bf16(tmp_path / "k.npy")
    assert np.array_equal(k, oracle.kv_append(kc, kn))
    assert cli("kv_cache_update", VC, VN, tmp_path / "v.npy").returncode == 0
    v = load_bf16(tmp_path / "v.npy")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = oracle.attention_prefill(q, k, v, scale, True)
    assert cli("attention_prefill", Q, tmp_path / "k.npy", tmp_path / "v.npy", tmp_path / "o.npy").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "o.npy"), want, rel_t=mt.LARGE_K_MAX_REL_ERR)
    assert cli("fused_kv_append_attention", Q, KC, VC, KN, VN, tmp_path / "fo.npy",
               "--kc-out", tmp_path / "kc2.npy").returncode == 0
    mt.assert_correct(load_bf16(tmp_path / "fo.npy"), want, rel_t=mt.LARGE_K_MAX_REL_ERR)
    assert np.array_equal(load_bf16(tmp_path / "kc2.npy"), k)  # the in-place append, bit-exact
