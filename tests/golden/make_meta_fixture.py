"""Writes tests/golden/meta_step_small.npz: input/output vectors of the
reference TTT model's meta step, for the harness in ttt_e2e/ (model.py,
meta.py), which nothing else ties to the reference.

The reference package (cloud_ttt_e2e/ttt_e2e: model.py:9-143,
meta.py:140-177, data.py, and its own torch attention, attention.py:9-131) is
imported from /root/reference and run on the CPU in float64:
  inputs   the model's initial parameters (torch.manual_seed(0)) and one
           key-value batch from the reference's generator;
  outputs  the inner and outer losses of meta_step and the gradient of the
           outer loss with respect to every parameter.
Configuration: vocab 32, d_model 16, 2 heads, 3 layers (2 adapted),
d_ff 32, window 32, T 96 in chunks of 48, 2 inner steps of lr 0.1 on
mlp_fast.

Run in the build container (the reference is not on the GPU box):
    python tests/golden/make_meta_fixture.py
"""
import os
import sys

import numpy as np
import torch

REF = "/root/reference/cloud_ttt_e2e"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "meta_step_small.npz")

CFG = dict(vocab_size=32, max_seq_len=96, window_size=32, d_model=16, n_heads=2, n_layers=3, d_ff=32,
           suffix_layers=2, dual_mlp=True)
STEP = dict(inner_lr=0.1, inner_steps=2, param_filter="mlp_fast", chunk_size=48)
BATCH = dict(batch_size=2, context_len=60, query_len=30, num_keys=8, pad_to=96, far_frac=0.5)


def main():
    sys.path.insert(0, REF)
    from ttt_e2e import data as rdata  # the reference package
    from ttt_e2e import meta as rmeta
    from ttt_e2e import model as rmodel

    torch.manual_seed(0)
    model = rmodel.TTTModel(rmodel.ModelConfig(**CFG)).double()
    init = {n: p.detach().clone() for n, p in model.named_parameters()}
    bt = rdata.generate_kv_batch(BATCH["batch_size"], BATCH["context_len"], BATCH["query_len"], CFG["vocab_size"],
                                 num_keys=BATCH["num_keys"], device="cpu", pad_to=BATCH["pad_to"],
                                 far_frac=BATCH["far_frac"])
    inner, outer = rmeta.meta_step(model, bt.input_ids, bt.targets, bt.inner_mask.double(), bt.outer_mask.double(),
                                   **STEP)
    outer.backward()
    arrays = {"input_ids": bt.input_ids.numpy(), "targets": bt.targets.numpy(),
              "inner_mask": bt.inner_mask.double().numpy(), "outer_mask": bt.outer_mask.double().numpy(),
              "inner_loss": np.array(inner.item()), "outer_loss": np.array(outer.item())}
    for n, p in model.named_parameters():
        arrays["param/" + n] = init[n].numpy()
        arrays["grad/" + n] = (p.grad if p.grad is not None else torch.zeros_like(p)).numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: inner {inner.item():.6f} outer {outer.item():.6f}, {len(init)} parameters")


if __name__ == "__main__":
    main()
