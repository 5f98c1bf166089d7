"""The direct-resident GGUF loader on the device: a synthetic GGUF holding Q4_K, Q8_0 and
Q6_K matmul weights (and an F32 norm that stays on the host) is read, each quantized weight
is uploaded from its memory-mapped bytes, and the device copy is checked two ways: its
dequantization is bit-identical to the oracle's dequantization of the file's bytes, and its
matmul meets the GEMV bound (max|dY|/RMS <= 1e-3) against the oracle's row dot products."""
import numpy as np
import pytest

from fak_amd import gguf, synth
from fak_amd.gguf import TensorType
from tests import q6k_cases as qc
from tests.gpu_util import Dev, rel_err

pytestmark = pytest.mark.gpu

DEQUANT = {TensorType.Q4_K: "fhip_q4k_dequant_f32", TensorType.Q8_0: "fhip_q8_0_dequant_f32",
           TensorType.Q6_K: "fhip_q6k_dequant_f32"}


def model_file(path):
    rng = np.random.default_rng(11)
    q6 = qc.pin_d(rng.integers(0, 256, 24 * 2 * 210, dtype=np.uint8), 0x1400)
    tens = [("blk.0.ffn_gate.weight", [512, 48], TensorType.Q4_K, synth.q4k_weights(48, 512, 1)),
            ("blk.0.attn_q.weight", [256, 40], TensorType.Q8_0, synth.q8_0_weights(40, 256, 2)),
            ("output.weight", [512, 24], TensorType.Q6_K, q6),
            ("blk.0.attn_norm.weight", [512], TensorType.F32,
             rng.standard_normal(512).astype(np.float32).view(np.uint8))]
    gguf.write(path, [("general.architecture", gguf.ValueType.STRING, "qwen2")],
               [(n, d, t, np.asarray(r, np.uint8).tobytes()) for n, d, t, r in tens])


def oracle_rows(oracle_mod, typ, raw, out, in_, X, P):
    if typ == TensorType.Q4_K:
        return oracle_mod.q4k_gemm(raw, out, in_, X, P)
    if typ == TensorType.Q8_0:
        return oracle_mod.q8_0_gemm(raw, out, in_, X, P)
    return oracle_mod.q6k_gemm(raw, out, in_, X, P)


def oracle_dequant(oracle_mod, typ, raw, out, in_):
    fn = {TensorType.Q4_K: oracle_mod.q4k_dequant, TensorType.Q8_0: oracle_mod.q8_0_dequant,
          TensorType.Q6_K: oracle_mod.q6k_dequant}[typ]
    return fn(raw, out, in_).reshape(out, in_)


def test_load_resident_matches_oracle(hip, oracle_mod, tmp_path):
    path = str(tmp_path / "m.gguf")
    model_file(path)
    with gguf.WeightSource(path) as ws:
        res = gguf.load_resident(ws)
        try:
            assert sorted(res) == ["blk.0.attn_q.weight", "blk.0.ffn_gate.weight", "output.weight"]
            for name, w in res.items():
                out, in_ = w.shape
                raw = np.frombuffer(ws.tensor_bytes(name), np.uint8).copy()
                print(f"[gguf] {name} {w.type.name} out={out} in={in_}", flush=True)
                with Dev(out * in_ * 4) as dw:
                    hip.call(DEQUANT[w.type], dw.ptr, w.ptr, out, in_)
                    got = dw.to_host(np.float32).reshape(out, in_)
                want = oracle_dequant(oracle_mod, w.type, raw, out, in_)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
                P = 3
                X = synth.activations(P, in_, 7)
                with Dev.from_host(X) as dx, Dev(P * out * 4) as dy:
                    w.matmul(dx.ptr, dy.ptr, P)
                    Y = dy.to_host(np.float32).reshape(P, out)
                ref = oracle_rows(oracle_mod, w.type, raw, out, in_, X, P)
                assert rel_err(Y, ref) <= 1e-3, name
        finally:
            for w in res.values():
                w.free()


def test_load_resident_selects_names(hip, tmp_path):
    path = str(tmp_path / "m.gguf")
    model_file(path)
    with gguf.WeightSource(path) as ws:
        res = gguf.load_resident(ws, names={"output.weight", "blk.0.attn_norm.weight"})
        try:
            assert list(res) == ["output.weight"] and res["output.weight"].shape == [24, 512]
        finally:
            for w in res.values():
                w.free()


def test_q4_k_m_layer_fused_mlp(hip, oracle_mod, tmp_path):
    """A q4_k_m-style FFN block (Q4_K ffn_gate / ffn_up [I, H], Q6_K ffn_down [H, I]) read from a
    GGUF file, made resident straight from the mapped bytes and run through the fused decode MLP:
    within the GEMV bound (max|dY|/RMS <= 1e-3) of the oracle's denseSwiGLU chain on the file's
    own bytes, for one and three tokens."""
    H, I = 512, 1536
    rng = np.random.default_rng(23)
    down = qc.pin_d(rng.integers(0, 256, H * (I // 256) * 210, dtype=np.uint8), 0x1000)
    tens = [("blk.0.ffn_gate.weight", [H, I], TensorType.Q4_K, synth.q4k_weights(I, H, 41)),
            ("blk.0.ffn_up.weight", [H, I], TensorType.Q4_K, synth.q4k_weights(I, H, 42)),
            ("blk.0.ffn_down.weight", [I, H], TensorType.Q6_K, down)]
    path = str(tmp_path / "layer.gguf")
    gguf.write(path, [("general.architecture", gguf.ValueType.STRING, "qwen2")],
               [(n, d, t, np.asarray(r, np.uint8).tobytes()) for n, d, t, r in tens])
    with gguf.WeightSource(path) as ws:
        res = gguf.load_resident(ws)
        try:
            g, u, d = (res[f"blk.0.ffn_{k}.weight"] for k in ("gate", "up", "down"))
            assert g.shape == [I, H] and u.shape == [I, H] and d.shape == [H, I]
            assert d.type == TensorType.Q6_K
            raw = {k: np.frombuffer(ws.tensor_bytes(f"blk.0.ffn_{k}.weight"), np.uint8).copy()
                   for k in ("gate", "up", "down")}
            for P in (1, 3):
                print(f"[gguf] q4_k_m FFN H={H} I={I} P={P}", flush=True)
                X = synth.activations(P, H, 60 + P)
                with Dev.from_host(X) as dx, Dev(P * H * 4) as dy:
                    hip.call("fhip_q4k_mlp_q6down_f32", g.ptr, u.ptr, d.ptr, dx.ptr, dy.ptr, H, I, P)
                    Y = dy.to_host(np.float32).reshape(P, H)
                ref = oracle_mod.q4k_mlp(raw["gate"], raw["up"], raw["down"], H, I, X, P,
                                         down_q6=True, workers=8)
                assert np.all(np.isfinite(Y))
                assert rel_err(Y, ref) <= 1e-3, (P, rel_err(Y, ref))
        finally:
            for w in res.values():
                w.free()
