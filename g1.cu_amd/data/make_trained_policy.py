"""Convert the reference's trained PPO checkpoint (models/ppo_ckpt/finish_best.pt of Infatoshi/g1.cu)
into plain arrays: the packed policy vector in the kernel's order (body linears weight [out,in]
row-major + bias, mu weight/bias, v weight/bias, log_std; the reference's scripts/ppo_fused.py:35-44
order) and the frozen observation statistics saved with it. The checkpoint is read with
torch.load(weights_only=True) (no unpickling of code); the output is a NumPy .npz (no pickle).

    python g1.cu_amd/data/make_trained_policy.py /root/reference/models/ppo_ckpt/finish_best.pt
"""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "trained_policy_finish_best.npz")


def main():
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/models/ppo_ckpt/finish_best.pt"
    raw = open(src, "rb").read()
    ck = torch.load(src, map_location="cpu", weights_only=True)
    m = ck["model"]
    order = ["body.0.weight", "body.0.bias", "body.2.weight", "body.2.bias", "mu.weight", "mu.bias",
             "v.weight", "v.bias", "log_std"]
    W = np.concatenate([m[k].reshape(-1).numpy().astype(np.float32) for k in order])
    assert W.size == 256 * 100 + 256 + 256 * 256 + 256 + 29 * 256 + 29 + 256 + 1 + 29
    np.savez(OUT, W=W, obs_mean=ck["obs_mean"].numpy().astype(np.float32),
             obs_var=ck["obs_var"].numpy().astype(np.float32),
             source_sha256=np.frombuffer(hashlib.sha256(raw).hexdigest().encode(), np.uint8))
    print(OUT, W.size, "params; source sha256", hashlib.sha256(raw).hexdigest())


if __name__ == "__main__":
    main()
