"""Calibration workload for rocprofv3 byte counters: five device-to-device
copies of 256 MiB (each reads and writes exactly 268435456 bytes). Run it under
``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE``; the counter values of the
copy kernel give the counter-to-bytes factors used by ``rocprof_summary``."""
import torch

NBYTES = 256 << 20

if __name__ == "__main__":
    x = torch.ones(NBYTES // 4, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(f"copy calibration: {NBYTES} bytes read and written per dispatch", flush=True)
