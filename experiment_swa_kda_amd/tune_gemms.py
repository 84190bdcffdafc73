"""Writes gemm_selection_gfx950.csv, the library GEMM solutions that
model.use_tuned_gemms() selects for the trainer's shapes.

Runs eager forward + backward micro-steps of the 6-layer config-4 model (d_model 384,
vocab 32768, B2 T4096) with torch's TunableOp tuning enabled, so every projection, lm_head
and weight-gradient GEMM shape of the trainer is timed over the hipBLASLt and rocBLAS
solutions, and writes the winners.  Run on the target GPU with the same ROCm / torch
stack that will read the file (the file's validator lines record them):

    python -m experiment_swa_kda_amd.tune_gemms [output.csv]
"""

from __future__ import annotations

import os
import sys

import torch


def main(out: str) -> None:
    from .model import GPT, GPTConfig

    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_filename(os.path.abspath(out))  # TunableOp writes the table there at exit
    torch.manual_seed(0)
    cfg = GPTConfig(sequence_len=4096, vocab_size=32768, n_layer=6, n_head=3, n_embd=384)
    model = GPT(cfg).cuda()
    model.init_weights()
    ids = torch.randint(0, cfg.vocab_size, (2, 4097), device="cuda")
    for _ in range(2):
        loss = model(ids[:, :-1], ids[:, 1:])
        loss.backward()
        model.zero_grad(set_to_none=True)
    torch.cuda.synchronize()
    print(f"{len(tun.get_results())} GEMM selections; written to {out} at exit", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else
         os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_selection_gfx950.csv"))
