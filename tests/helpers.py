"""Shared data builders for the GPU parity tests (synthetic inputs as the
benchmark configs define them: codes uniform in [-8, 7] stored offset-8,
fp16 scales |N(0, 0.02)|, activations N(0, 1))."""
import numpy as np
import torch

from oracle import q4_oracle as O


def synth_int4(rng, N, K):
    """codes q (offset-8 uint8 [N, K]) and fp16 scales [N, K/32] as float32 values."""
    q = (rng.integers(-8, 8, (N, K)) + 8).astype(np.uint8)
    s = np.abs(rng.normal(0, 0.02, (N, K // 32))).astype(np.float16).astype(np.float32)
    return q, s


def upload_int4(q, s16, device="cuda"):
    """Host codes/fp16 scales -> device panel-64 words (int32) + fp16 panel scales."""
    words = O.pack_dev(q).view(np.int32)
    sc = O.scales_dev(np.asarray(s16, np.float32).astype(np.float16))
    return torch.from_numpy(words).to(device), torch.from_numpy(sc).to(device)


def to_np(t):
    return t.detach().cpu().numpy()


def sync():
    torch.cuda.synchronize()
