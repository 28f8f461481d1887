"""Write the golden fixtures that pin the oracle to the reference implementation.

Run in the build container only (the reference checkout is not present on
the GPU box):

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py

It imports the reference's pure-PyTorch ``moe_backend="pytorch"`` path from
``/root/reference`` (read-only), runs it on CPU in fp32 and stores inputs and
outputs as small ``.npz`` files next to this script.  Nothing of the reference
itself is stored: only parameter hashes, input ids and output tensors.

What is pinned here (nothing else in the reference pins it):
  * seed-0 parameter initialisation of the tiny config (per-parameter SHA-256
    of the fp32 bytes), which depends on module registration order
    (reference parrot/model.py:639-656);
  * full forward of the tiny config: logits summary, per-layer router logits,
    top-2 indices and weights, per-layer MoE input/output, depth-mix outputs
    (reference parrot/model.py:505-569, 658-746);
  * prefill + cached decode logits (reference parrot/model.py:748-931);
  * the tie behaviour of ``torch.topk`` on exactly equal probabilities
    (reference parrot/model.py:526).
"""
import hashlib
import os
import sys
from dataclasses import replace
from pathlib import Path

import numpy as np
import torch
from torch.nn import functional as F

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent

# The tiny configuration: the reference README names an `example.py --tiny`
# config that is absent from its snapshot; this definition is the build's own.
TINY = dict(
    vocab_size=32768, dim=64, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=16,
    kv_latent_dim=32, window_size=32, max_seq_len=128, local_query_chunk=16,
    n_experts=8, expert_dim=128, shared_expert_dim=64,
)
SLICE = 256  # logits columns stored verbatim


def _logit_summary(prefix, logits):
    logits = logits.detach().float()
    flat = logits.reshape(-1, logits.shape[-1])
    top_v, top_i = flat.topk(8, dim=-1)
    return {
        f"{prefix}_argmax": flat.argmax(-1).numpy().astype(np.int64),
        f"{prefix}_lse": torch.logsumexp(flat, -1).numpy(),
        f"{prefix}_top8_values": top_v.numpy(),
        f"{prefix}_top8_ids": top_i.numpy().astype(np.int64),
        f"{prefix}_slice": flat[:, :SLICE].numpy(),
    }


def main():
    sys.path.insert(0, str(REFERENCE))
    os.environ.setdefault("PYTHONDONTWRITEBYTECODE", "1")
    from parrot import ModelConfig, Parrot  # the reference package

    torch.set_num_threads(4)
    cfg = ModelConfig(**TINY)

    # ---- 1. seed-0 initialisation ------------------------------------------
    torch.manual_seed(0)
    model = Parrot(cfg).eval()
    names, shapes, digests = [], [], []
    for name, param in model.state_dict().items():
        names.append(name)
        shapes.append(",".join(str(s) for s in param.shape))
        digests.append(hashlib.sha256(
            param.detach().float().contiguous().numpy().tobytes()).hexdigest())
    np.savez(OUT / "tiny_init.npz", names=np.array(names), shapes=np.array(shapes),
             sha256=np.array(digests))

    # ---- 2. full forward with hooks ----------------------------------------
    ids = torch.randint(0, cfg.vocab_size, (1, 64),
                        generator=torch.Generator().manual_seed(0))
    moe_in, moe_out, depth_out = {}, {}, {}

    def moe_pre(idx):
        def hook(module, args):
            moe_in[idx] = args[0].detach().clone()
        return hook

    def moe_post(idx):
        def hook(module, args, output):
            moe_out[idx] = output[0].detach().clone()
        return hook

    def depth_post(idx):
        def hook(module, args, output):
            depth_out[idx] = output.detach().clone()
        return hook

    handles = []
    for i, block in enumerate(model.blocks):
        handles.append(block.moe.register_forward_pre_hook(moe_pre(i)))
        handles.append(block.moe.register_forward_hook(moe_post(i)))
    for j, mix in enumerate(model.depth_mix):
        handles.append(mix.register_forward_hook(depth_post(j)))
    with torch.no_grad():
        out = model(ids)
    for h in handles:
        h.remove()

    L = cfg.n_layers
    router_logits, top_idx, top_w = [], [], []
    torch.set_grad_enabled(False)
    for i in range(L):
        flat = moe_in[i].reshape(-1, cfg.dim)
        logits = F.linear(flat.float(), model.blocks[i].moe.router.weight.float())
        probs = logits.softmax(-1)
        w, idx = probs.topk(cfg.top_k, dim=-1)
        w = w / w.sum(-1, keepdim=True)
        router_logits.append(logits.numpy())
        top_idx.append(idx.numpy().astype(np.int64))
        top_w.append(w.numpy())
    forward = {
        "ids": ids.numpy().astype(np.int64),
        "router_logits": np.stack(router_logits),
        "top2_indices": np.stack(top_idx),
        "top2_weights": np.stack(top_w),
        "moe_input": np.stack([moe_in[i].reshape(-1, cfg.dim).numpy() for i in range(L)]),
        "moe_output": np.stack([moe_out[i].reshape(-1, cfg.dim).numpy() for i in range(L)]),
        "depth_output": np.stack([depth_out[j].reshape(-1, cfg.dim).numpy()
                                  for j in range(2 * L + 1)]),
    }
    forward.update(_logit_summary("logits", out.logits))
    np.savez(OUT / "tiny_forward.npz", **forward)

    # ---- 3. forward with router stats (aux loss / utilisation) -------------
    with torch.no_grad():
        out_stats = model(ids, labels=ids)
    np.savez(OUT / "tiny_forward_stats.npz",
             aux_loss=np.array(out_stats.aux_loss.item(), dtype=np.float32),
             lm_loss=np.array(out_stats.lm_loss.item(), dtype=np.float32),
             loss=np.array(out_stats.loss.item(), dtype=np.float32),
             expert_utilization=out_stats.expert_utilization.numpy())

    # ---- 4. standard residual variant ---------------------------------------
    torch.manual_seed(0)
    std_model = Parrot(replace(cfg, residual="standard")).eval()
    with torch.no_grad():
        std_out = std_model(ids)
    np.savez(OUT / "tiny_forward_standard.npz", **_logit_summary("logits", std_out.logits))

    # ---- 5. prefill + cached decode (batch 2, crosses the local window) -----
    prompt = torch.randint(0, cfg.vocab_size, (2, 40),
                           generator=torch.Generator().manual_seed(3))
    gen = {"prompt": prompt.numpy().astype(np.int64)}
    logits, state = model.prefill(prompt)
    gen.update(_logit_summary("prefill", logits))
    step_ids = []
    steps = []
    for step in range(6):
        next_id = logits[:, -1].argmax(-1, keepdim=True)
        step_ids.append(next_id.numpy().astype(np.int64))
        logits, state = model.decode_step(next_id, state)
        steps.append(_logit_summary("s", logits))
    gen["decode_ids"] = np.stack(step_ids)
    for key in steps[0]:
        gen["decode" + key[1:]] = np.stack([s[key] for s in steps])
    gen["final_position"] = np.array(state.position, dtype=np.int64)
    np.savez(OUT / "tiny_generate.npz", **gen)

    # ---- 6. torch.topk tie behaviour on equal probabilities ----------------
    tie_logits = torch.tensor([
        [0.5, 0.5, 0.1, 0.1, 0.0, 0.0, 0.0, 0.0],
        [0.1, 0.3, 0.3, 0.3, 0.0, 0.0, 0.0, 0.0],
        [1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0],
        [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.7, 0.7],
        [0.2, 0.9, 0.2, 0.9, 0.2, 0.9, 0.2, 0.9],
        [-1.0, -2.0, -1.0, -3.0, -2.0, -1.0, -4.0, -5.0],
    ], dtype=torch.float32)
    probs = tie_logits.softmax(-1)
    w, idx = probs.topk(2, dim=-1)
    np.savez(OUT / "topk_ties.npz", logits=tie_logits.numpy(),
             indices=idx.numpy().astype(np.int64),
             weights=(w / w.sum(-1, keepdim=True)).numpy())
    print("wrote fixtures to", OUT)


if __name__ == "__main__":
    main()
