"""Synthetic MoE model files for tests: a qwen3moe-named GGUF with expert
stacks (Q4_K gate/up, Q6_K down) in GGUF layout, F32 routers and norms, an
optional shared expert per layer and a Q6_K LM head; returns the host arrays
it wrote."""
import numpy as np

import gguf_writer as W
import kq_synth as S

Q4_K, Q6_K = 12, 14
EPS = 1e-6


def build_gguf(path, L=2, hidden=1024, ffn=512, E=16, n_sel=4, shared=(1,), vocab=3000, seed=0):
    rng = np.random.default_rng(seed)
    w = W.GgufWriter(alignment=32)
    w.kv("general.architecture", W.STR, "qwen3moe").kv("qwen3moe.block_count", W.U32, L)
    w.kv("qwen3moe.embedding_length", W.U32, hidden).kv("qwen3moe.expert_count", W.U32, E)
    w.kv("qwen3moe.expert_used_count", W.U32, n_sel).kv("qwen3moe.attention.layer_norm_rms_epsilon", W.F32, EPS)
    host = {"layers": []}
    for li in range(L):
        g = S.matrix(rng, Q4_K, E * ffn, hidden)
        u = S.matrix(rng, Q4_K, E * ffn, hidden)
        d = S.matrix(rng, Q6_K, E * hidden, ffn)
        router = (rng.standard_normal((E, hidden)) * 0.05).astype(np.float32)
        norm = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
        w.tensor(f"blk.{li}.ffn_gate_exps.weight", [hidden, ffn, E], Q4_K, g)
        w.tensor(f"blk.{li}.ffn_up_exps.weight", [hidden, ffn, E], Q4_K, u)
        w.tensor(f"blk.{li}.ffn_down_exps.weight", [ffn, hidden, E], Q6_K, d)
        w.tensor(f"blk.{li}.ffn_gate_inp.weight", [hidden, E], 0, router)
        w.tensor(f"blk.{li}.ffn_norm.weight", [hidden], 0, norm)
        sh = None
        if li in shared:
            sh = (ffn, S.matrix(rng, Q4_K, ffn, hidden), S.matrix(rng, Q4_K, ffn, hidden),
                  S.matrix(rng, Q6_K, hidden, ffn))
            w.tensor(f"blk.{li}.ffn_gate_shexp.weight", [hidden, ffn], Q4_K, sh[1])
            w.tensor(f"blk.{li}.ffn_up_shexp.weight", [hidden, ffn], Q4_K, sh[2])
            w.tensor(f"blk.{li}.ffn_down_shexp.weight", [ffn, hidden], Q6_K, sh[3])
        host["layers"].append(dict(g=g, u=u, d=d, router=router, norm=norm, sh=sh))
    host["out_norm"] = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    host["head"] = S.matrix(rng, Q6_K, vocab, hidden)
    w.tensor("output_norm.weight", [hidden], 0, host["out_norm"])
    w.tensor("output.weight", [hidden, vocab], Q6_K, host["head"])
    w.write(path)
    host.update(L=L, hidden=hidden, ffn=ffn, E=E, n_sel=n_sel, vocab=vocab)
    return host
