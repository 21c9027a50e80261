"""Writes the golden fixtures of tests/golden/ from the REFERENCE's own CPU code.

Runs oracle/_ref/ref_harness (the reference's src/{tensor,common_ops,
transformer_ops,transformer,scheduler,torch_rng}.cpp compiled from
/root/reference by oracle/ref/Makefile) on the seeded synthetic model of
oracle/model_spec.h and stores, per output tensor, its SHA-256 over the fp32
bytes, its L2 norm, a strided subsample and (when small) the whole tensor;
a tensor too large to store whole also gets a spread subsample: the values
at flat indices (k * SPREAD_STEP) mod size, k < SPREAD, which (SPREAD_STEP odd,
prime and coprime with every size here) land on SPREAD distinct indices
spread over every row and column rather than on one column as a stride
that divides the row length does.
Only data goes into the fixtures; nothing of the reference's source does.

Cases (one .npz each):
  cfg1_self16  single block, 16x16 tokens, t=500, self heads 16x72
  cfg1_self36  same with the production 36x32 self heads
  cfg2         full 28-block forward at 1024 px, t=999, no mask, and the
               reference's own run_full_denoising_step_with_cfg step 0
               (checked bit-exact against forward + CFG + scheduler)
  cfg2_mask    same forward with the Gemma padding mask (1 / 40 real tokens)
  cfg3         20-step DPM-Solver++ loop, guidance 4.5, final latent
  nonsquare    full 28-block forward on a 4x16 latent (64 tokens, which the
               reference runs through each block's depthwise conv as an 8x8
               grid), t=999, no mask
  cfg5         full 28-block forward at 4096 px (latent 128x128, 16384
               tokens), t=999, no mask
  vae_small    the reference's run_vae_decode on the small synthetic DC-AE
               decoder of oracle/vae_spec.h, latent 8x8 -> 64x64 RGB
  vae_conv     both summation orders of the reference's 3x3 conv
               (conv2d_3x3_im2col_gemm, conv2d_3x3_tap_accumulate)
  vae_full     run_vae_decode on the full Sana 1.0 DC-AE f32c32 decoder,
               latent 32x32 -> 1024x1024 RGB
  vae_weights  64-bit FNV-1a digest of every synthetic VAE weight (small, full)
  weights      64-bit FNV-1a digest of every generated weight tensor (the
               reference's randn_torch_cpu, seed 1000 + sorted index)

usage: python tests/golden/make_golden.py [case ...]   (default: all)
"""
import hashlib
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(ROOT, "oracle", "_ref", "ref_harness")

CASES = {
    "cfg1_self16": (["block", "16", "16", "16", "500"],
                    {"x": (1, 256, 1152), "t_mod": (1, 6912), "after_self": (1, 256, 1152),
                     "after_cross": (1, 256, 1152), "after_ff": (1, 256, 1152)}),
    "cfg1_self36": (["block", "36", "16", "16", "500"],
                    {"x": (1, 256, 1152), "t_mod": (1, 6912), "after_self": (1, 256, 1152),
                     "after_cross": (1, 256, 1152), "after_ff": (1, 256, 1152)}),
    "cfg2": (["forward", "36", "16", "32", "999", "0", "1"],
             {"context": (2, 300, 1152), "noise_pred": (2, 32, 32, 32), "guided": (1, 32, 32, 32),
              "step0": (1, 32, 32, 32)}),
    "cfg2_mask": (["forward", "36", "16", "32", "999", "1", "0"],
                  {"context": (2, 300, 1152), "noise_pred": (2, 32, 32, 32), "guided": (1, 32, 32, 32)}),
    "cfg3": (["loop", "36", "16", "32", "20", "4.5", "0"], {"final_latent": (1, 32, 32, 32)}),
    "nonsquare": (["forward-hw", "36", "16", "4", "16", "999"], {"noise_pred": (2, 32, 4, 16)}),
    "cfg5": (["forward", "36", "16", "128", "999", "0", "0"],
             {"context": (2, 300, 1152), "noise_pred": (2, 32, 128, 128), "guided": (1, 32, 128, 128)}),
    "vae_small": (["vae", "small", "8"],
                  {"latent": (1, 32, 8, 8), "decoder_input": (1, 128, 8, 8), "image": (1, 3, 64, 64)}),
    "vae_conv": (["vae-conv", "13", "24", "40"],
                 {"x": (1, 24, 13, 13), "w": (40, 24, 3, 3), "bias": (40,), "im2col": (1, 40, 13, 13),
                  "tap": (1, 40, 13, 13)}),
    "vae_full": (["vae", "full", "32"],
                 {"latent": (1, 32, 32, 32), "decoder_input": (1, 1024, 32, 32), "image": (1, 3, 1024, 1024)}),
}
FULL_LIMIT = 70000      # tensors up to this many values are stored whole
SUBSAMPLE = 4096
SPREAD = 65536
SPREAD_STEP = 1000003


def weights():
    res = subprocess.run([EXE, "digest"], capture_output=True, text=True, check=True)
    names, digests = [], []
    for ln in res.stdout.splitlines():
        n, h = ln.split()
        names.append(n)
        digests.append(int(h, 16))
    np.savez_compressed(os.path.join(HERE, "weights.npz"), names=np.array(names),
                        fnv1a=np.array(digests, dtype=np.uint64))
    print("wrote weights:", len(names), "tensors", flush=True)


def vae_weights():
    out = {}
    for which in ("small", "full"):
        res = subprocess.run([EXE, "vae-digest", which], capture_output=True, text=True, check=True)
        names, digests = [], []
        for ln in res.stdout.splitlines():
            n, h = ln.split()
            names.append(n)
            digests.append(int(h, 16))
        out[which + "_names"] = np.array(names)
        out[which + "_fnv1a"] = np.array(digests, dtype=np.uint64)
    np.savez_compressed(os.path.join(HERE, "vae_weights.npz"), **out)
    print("wrote vae_weights", flush=True)


def main(names):
    if not os.path.exists(EXE):
        sys.exit(f"{EXE} missing: build it with `make -C oracle/ref` (needs /root/reference)")
    for name in names:
        if name == "weights":
            weights()
            continue
        if name == "vae_weights":
            vae_weights()
            continue
        args, tensors = CASES[name]
        with tempfile.TemporaryDirectory() as tmp:
            cmd = [EXE] + args + [tmp]
            print("running", " ".join(cmd), flush=True)
            res = subprocess.run(cmd, capture_output=True, text=True)
            print(res.stdout, res.stderr, flush=True)
            if res.returncode != 0:
                sys.exit(f"{name}: reference harness failed")
            out = {"args": np.array(args)}
            for tn, shape in tensors.items():
                a = np.fromfile(os.path.join(tmp, tn + ".f32"), dtype=np.float32)
                assert a.size == int(np.prod(shape)), (tn, a.size, shape)
                a = a.reshape(shape)
                out[tn + "__sha256"] = np.array(hashlib.sha256(a.tobytes()).hexdigest())
                out[tn + "__l2"] = np.array(np.linalg.norm(a.astype(np.float64)))
                stride = max(1, a.size // SUBSAMPLE)
                out[tn + "__stride"] = np.array(stride)
                out[tn + "__sub"] = a.reshape(-1)[::stride].copy()
                if a.size <= FULL_LIMIT:
                    out[tn] = a
                else:
                    idx = (np.arange(SPREAD, dtype=np.int64) * SPREAD_STEP) % a.size
                    assert np.unique(idx).size == SPREAD
                    out[tn + "__spread_step"] = np.array(SPREAD_STEP)
                    out[tn + "__spread"] = a.reshape(-1)[idx].copy()
            for ln in res.stdout.splitlines():
                if ln.endswith("_ms") or "_ms " in ln:
                    k, v = ln.split()[:2]
                    out["ref_" + k] = np.array(float(v))
            np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
            print("wrote", name, flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or list(CASES) + ["weights", "vae_weights"])
