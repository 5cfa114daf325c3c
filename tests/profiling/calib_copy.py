#!/usr/bin/env python3
"""Calibration workload for HBM byte counters: copies a 1 GiB device buffer
into another 1 GiB buffer (torch's copy kernel) a few times.  Each copy reads
2^30 bytes and writes 2^30 bytes, so FETCH_SIZE / WRITE_SIZE per dispatch
divided by 2^20 KiB is the scale factor of those counters."""
import torch

n = (1 << 30) // 4
src = torch.ones(n, dtype=torch.int32, device="cuda")
dst = torch.empty_like(src)
torch.cuda.synchronize()
for _ in range(5):
    dst.copy_(src)
torch.cuda.synchronize()
print("calibration copies done: 5 x 1 GiB", flush=True)
