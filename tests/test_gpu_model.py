"""A two-layer model end to end, the way the engine drives the device path:
a GGUF file (Q8_0 token embedding, Q4_K_M layers, F32 norms, Q6_K output
head) written by the test writer, read and uploaded through the library's
GGUF reader, a 24-token prompt through dq_layer_prefill layer by layer, the
head and a greedy draw on the device, then two decode steps whose x is built
on the device from the drawn token. Against the oracle's chain of the same
steps: the logits of every step within the layer tolerance, and the same
tokens wherever the oracle's top-two margin exceeds that noise."""
import numpy as np
import pytest
import torch

from desireeia_amd import gguf, ops, synth
from oracle.oracle import LayerArgs

import gguf_writer as gw

pytestmark = pytest.mark.gpu
E, H, KV, HD, F, V, NL = 512, 8, 2, 128, 1024, 3000, 2
TOL_LOGITS = 3e-2  # the oracle's own logits move ~2e-2 under 4e-4 product errors (test_oracle_sensitivity.py)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def build_file(path):
    rng = np.random.default_rng(1)
    tensors, raw = [], {}

    def add(name, qtype, rows, cols, data=None):
        if data is None:
            data = synth.gen_weights(qtype, rows, cols, seed=len(tensors) + 10)
        raw[name] = np.ascontiguousarray(data)
        tensors.append((name, qtype, [cols, rows] if rows > 1 else [cols], raw[name].tobytes()))

    add("token_embd.weight", synth.Q8_0, V, E)
    for l in range(NL):
        p = f"blk.{l}."
        add(p + "attn_norm.weight", 0, 1, E, (0.25 / np.sqrt(E) * (1 + 0.02 * rng.standard_normal(E))).astype(np.float32))
        add(p + "attn_q.weight", synth.Q4_K, H * HD, E)
        add(p + "attn_k.weight", synth.Q4_K, KV * HD, E)
        add(p + "attn_v.weight", synth.Q6_K, KV * HD, E)
        add(p + "attn_output.weight", synth.Q4_K, E, H * HD)
        add(p + "ffn_norm.weight", 0, 1, E, (0.3 / np.sqrt(E) * (1 + 0.02 * rng.standard_normal(E))).astype(np.float32))
        add(p + "ffn_gate.weight", synth.Q4_K, F, E)
        add(p + "ffn_up.weight", synth.Q4_K, F, E)
        add(p + "ffn_down.weight", synth.Q6_K, E, F)
    add("output_norm.weight", 0, 1, E, (1 + 0.05 * rng.standard_normal(E)).astype(np.float32))
    add("output.weight", synth.Q6_K, V, E)
    kv = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.U32, NL),
          ("llama.embedding_length", gw.U32, E), ("llama.feed_forward_length", gw.U32, F),
          ("llama.attention.head_count", gw.U32, H), ("llama.attention.head_count_kv", gw.U32, KV),
          ("llama.rope.freq_base", gw.F32, 500000.0), ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5)]
    gw.write_gguf(path, kv, tensors)
    return raw


def test_two_layer_model(gpu, orc, tmp_path):
    path = tmp_path / "tiny.gguf"
    raw = build_file(path)
    T, n_ctx = 24, 40
    prompt = np.random.default_rng(2).integers(0, V, T).astype(np.int32)
    with gguf.GgufFile(path) as f:
        assert f.get("llama.block_count") == NL and f.get("llama.embedding_length") == E
        theta = f.get("llama.rope.freq_base")
        eps = f.get("llama.attention.layer_norm_rms_epsilon")
        emb = f.matrix("token_embd.weight")
        head = f.matrix("output.weight")
        onorm = torch.from_numpy(f.read_tensor_raw("output_norm.weight")[0].view(np.float32).copy()).to(gpu)
        layers, oargs = [], []
        for l in range(NL):
            p = f"blk.{l}."
            mats = {nm: f.matrix(p + key) for nm, key in (("q", "attn_q.weight"), ("k", "attn_k.weight"),
                                                         ("v", "attn_v.weight"), ("o", "attn_output.weight"),
                                                         ("gate", "ffn_gate.weight"), ("up", "ffn_up.weight"),
                                                         ("down", "ffn_down.weight"))}
            an = torch.from_numpy(f.read_tensor_raw(p + "attn_norm.weight")[0].view(np.float32).copy())
            fn = torch.from_numpy(f.read_tensor_raw(p + "ffn_norm.weight")[0].view(np.float32).copy())
            layers.append(ops.DecoderLayer(mats, an, fn, H, KV, HD, n_ctx, rms_eps=eps, rope_theta=theta, device=gpu))
            a = LayerArgs(E, H, KV, HD, F, eps, theta, synth.Q4_K, synth.Q4_K, synth.Q6_K, synth.Q4_K, synth.Q4_K,
                          synth.Q4_K, synth.Q6_K)
            for nm, key in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                            ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                setattr(a, "w" + nm, raw[p + key + ".weight"].ctypes.data)
            a.attn_norm = raw[p + "attn_norm.weight"].ctypes.data
            a.ffn_norm = raw[p + "ffn_norm.weight"].ctypes.data
            oargs.append(a)
    # ---- the device chain
    tok = torch.from_numpy(prompt).to(gpu)
    x = torch.stack([ops.embed_q8_0(emb, tok[i:i + 1]) for i in range(T)])
    for L in layers:
        x = L.prefill(x, 0)
    dev_logits, dev_tokens = [], []
    logits = ops.head_logits(head, x[T - 1].contiguous(), onorm, eps)
    for step in range(3):
        dev_logits.append(logits.cpu().numpy())
        nxt, _ = ops.topk(logits, 1)
        dev_tokens.append(int(nxt.cpu()[0]))
        if step == 2:
            break
        xt = ops.embed_q8_0(emb, nxt)
        for L in layers:
            xt = L.decode(xt, T + step)
        logits = ops.head_logits(head, xt, onorm, eps)
    # ---- the oracle chain (its own cache)
    pb = KV * HD // 32 * 34
    caches = [(np.zeros(n_ctx * pb, np.uint8), np.zeros(n_ctx * pb, np.uint8)) for _ in range(NL)]
    E_rows = raw["token_embd.weight"]
    embed = lambda t: orc.dequantize_row(synth.Q8_0, np.ascontiguousarray(E_rows[t]), E)
    on = raw["output_norm.weight"]
    hx = np.stack([embed(t) for t in prompt])
    for a, (kc, vc) in zip(oargs, caches):
        hx = orc.layer_prefill(a, kc, vc, 0, hx)
    ref_logits = orc.matmul(synth.Q6_K, raw["output.weight"], V, E, orc.rms_norm(hx[T - 1], on, eps))
    tokens_checked = 0
    for step in range(3):
        e = rel(dev_logits[step], ref_logits)
        top2 = np.sort(ref_logits)[-2:]
        margin = (top2[1] - top2[0]) / max(np.abs(ref_logits).max(), 1e-30)
        print(f"  step {step}: logits rel {e:.2e}, token dev {dev_tokens[step]} oracle {int(np.argmax(ref_logits))} "
              f"(margin {margin:.3f})", flush=True)
        assert e <= TOL_LOGITS
        if margin > 2 * TOL_LOGITS:
            assert dev_tokens[step] == int(np.argmax(ref_logits))
            tokens_checked += 1
        if step == 2:
            break
        # the oracle continues from the device's token so both chains see the same inputs
        hxt = embed(dev_tokens[step])
        for a, (kc, vc) in zip(oargs, caches):
            hxt = orc.layer_decode(a, kc, vc, T + step, hxt)[0]
        ref_logits = orc.matmul(synth.Q6_K, raw["output.weight"], V, E, orc.rms_norm(hxt, on, eps))
    print(f"  tokens compared: {tokens_checked} of 3", flush=True)
