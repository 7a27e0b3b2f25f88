"""Write golden vectors from the reference's own HIP kernels (run on an MI355X).

Runs HipGPT's launch_multihead_attention, built from its sources by
`make -C oracle ref` into oracle/_ref/libref_hip_kernels.so, on planar inputs
regenerated from a seed (SplitMix64 -> Box-Muller, oracle/attn_oracle.c), and
stores the reference's O and P.  The shapes cover both reference kernels:
flash_attention_kernel<32|64> (D in {32, 64}, S <= 512) and the fallback
(other D, or S > 512).  Inputs are not stored: the seed and a checksum are.

Usage (GPU box, repo root):  python tests/golden/make_golden.py [OUTDIR]
(OUTDIR defaults to this directory, where the committed fixtures live.)
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402  (first: one HIP runtime for the process)

import oracle as O  # noqa: E402

# (B, S, E, H): flash D=32, flash D=64, fallback D=48, fallback D=128,
# fallback D=256, flash at S=1, fallback at S=513 (D=32 past the S<=512 cap).
SHAPES = [(1, 7, 64, 2), (2, 33, 128, 2), (1, 40, 96, 2), (1, 24, 256, 2), (1, 20, 256, 1),
          (1, 1, 32, 1), (1, 513, 32, 1)]
MAX_P = 1 << 16  # store full probs up to this many elements, else sampled rows


def main(outdir):
    os.makedirs(outdir, exist_ok=True)
    ref = O.ref_lib()
    for i, (B, S, E, H) in enumerate(SHAPES):
        seed = 0x474F4C44 + i
        qkv = O.seeded_planar(seed, B, S, E)
        d_qkv = torch.from_numpy(qkv).cuda()
        d_out = torch.zeros(B * S, E, device="cuda")
        d_p = torch.zeros(B, H, S, S, device="cuda")
        ref.launch(d_qkv.data_ptr(), d_out.data_ptr(), d_p.data_ptr(), B, S, E, H)
        torch.cuda.synchronize()
        out = d_out.cpu().numpy()
        probs = d_p.cpu().numpy()
        rows = np.arange(S)
        if probs.size > MAX_P:
            rows = np.unique(np.array([0, 1, S // 2, S - 2, S - 1]))
            probs = probs[:, :, rows, :]
        name = os.path.join(outdir, f"ref_B{B}_S{S}_E{E}_H{H}.npz")
        np.savez_compressed(name, B=B, S=S, E=E, H=H, seed=seed,
                            qkv_sum=np.float32(qkv.astype(np.float64).sum()),
                            out=out, probs=probs, prob_rows=rows)
        print("wrote", name, out.shape, probs.shape, flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.dirname(os.path.abspath(__file__)))
