"""Shared MoE edge-case material for the GPU tests and the oracle's own tests: the model spec, the
token sequence, NaN poisoning of chosen experts in a GGUF file, and the experts the oracle routes to."""
import numpy as np

import oracle as O
from sardyne_amd.gguf_synth import ModelSpec, read_tensors

F16_NAN = np.array([0x7E00], np.uint16).view(np.uint8).tobytes()
SCALE_BYTES = {12: (0, 2), 14: (208,), 8: (0,), 2: (0,), 6: (0,)}  # ggml type -> offsets of its f16 scales
BLOCK = {12: (256, 144), 14: (256, 210), 8: (32, 34), 2: (32, 18), 6: (32, 22)}

MOE = ModelSpec(arch="qwen3moe", n_vocab=300, dim=256, n_layer=2, n_head=4, n_kv_head=2, head_dim=64, ffn_dim=1024,
                context=64, n_expert=64, n_expert_used=2, ffn_exp_dim=256, qkv_bias=False, qk_norm=True,
                router_std=0.3)
PROMPT = list(np.random.default_rng(21).integers(0, 300, 16))  # one 16-token chunk: the GEMM threshold
STEPS = [5, 77, 140, 9]


def poison_experts(path, experts_per_layer):
    """Overwrites, in place, the f16 scales of every block of the given experts' gate, up and down rows
    with NaN (experts_per_layer[l]: expert indices of layer l)."""
    _, tensors, data_off, _ = read_tensors(path)
    mm = np.memmap(path, np.uint8, mode="r+")
    for l, experts in enumerate(experts_per_layer):
        experts = list(experts)
        if not experts:
            continue
        for g in ("gate", "up", "down"):
            ne, tid, off = tensors[f"blk.{l}.ffn_{g}_exps.weight"]
            per, bb = BLOCK[tid]
            blocks = mm[data_off + off:data_off + off + ne[2] * ne[1] * (ne[0] // per) * bb]
            blocks = blocks.reshape(ne[2], -1, bb)  # [expert][blocks of its rows][block bytes]
            for so in SCALE_BYTES[tid]:
                blocks[experts, :, so:so + 2] = np.frombuffer(F16_NAN, np.uint8)
    mm.flush()
    del mm


def used_experts(path):
    """Experts the oracle routes to for the prompt and the steps, per layer."""
    ref = O.OracleContext(path, 48, n_batch=16)
    ref.eval(PROMPT)
    used = [set(x.ravel().tolist()) for x in ref.last_topk(len(PROMPT))]
    for t in STEPS:
        ref.eval([t])
        for l, x in enumerate(ref.last_topk(1)):
            used[l].update(x.ravel().tolist())
    return used
