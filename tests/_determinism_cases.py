"""Output hashes of one product per launch regime, from seeded inputs (used by
tests/test_gpu_determinism.py in the test process and in a child process)."""
import hashlib
import json
import sys

import torch

# (M, N, K, G): decode M=1 (one-CU tiles and narrowed lone tiles), factored
# decode M=4/16, 32/64-row prefill tiles with split-K (M=32/64), skinny
# split-K (K % 64 != 0), prefill with split-K (M=128) and without (M=2048),
# the few-tile prefill kernel's K split across workgroups (M=128 with
# K=8192, M=512 with N=512, and 128 x 128 tiles for M=512 with K=8192), and
# the main prefill kernel's two K splits finished in the kernel (M=2048 with
# K=8192)
CASES = [(1, 2048, 2048, 128), (1, 2048, 8192, 128), (4, 512, 2048, 64), (16, 2048, 2048, 32),
         (32, 8192, 2048, 128), (64, 2048, 8192, 128), (40, 1024, 1032, 8), (128, 2048, 2048, 128),
         (2048, 2048, 2048, 128), (128, 2048, 8192, 128), (512, 512, 2048, 128), (512, 2048, 8192, 128),
         (2048, 2048, 8192, 128)]


def hashes() -> dict:
    import int4_hip
    out = {}
    for M, N, K, G in CASES:
        g = torch.Generator().manual_seed(M * 7919 + N * 31 + K + G)
        w = (torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16).cuda()
        x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
        qw, s, z = int4_hip.quantize_int4(w, G)
        y = int4_hip.w4a16_matmul(x, qw, s, z)
        torch.cuda.synchronize()
        h = hashlib.sha256()
        for t in (qw, s, z, y):
            h.update(t.cpu().contiguous().view(torch.uint8).numpy().tobytes())
        out[f"{M}x{N}x{K}/G{G}"] = h.hexdigest()
    return out


if __name__ == "__main__":
    sys.stdout.write(json.dumps(hashes()) + "\n")
