"""Runs the reference engine builds of oracle/_ref (see oracle/Makefile) on a synthetic model, for the e2e tests."""
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
REF = os.path.join(ROOT, "oracle", "_ref")
JOINT = 640


def binary(name):
    return os.path.join(REF, name)


def have(*names):
    return all(os.access(binary(n), os.X_OK) for n in names)


def env_for(mode):
    """Environment of an engine run: mode "exact-chain" is exact mode with the GPU's five-value exact route on the
    reference's per-output fmaf chain (P2H_EXACT_CHAIN=1), "exact" on the fp32 matrix cores."""
    e = dict(os.environ)
    for k in ("P2_GEMM", "P2_EXACT", "P2_CACHE_CODES", "P2H_EXACT_CHAIN"):
        e.pop(k, None)
    e["P2_THREADS"] = "8"
    if mode in ("exact", "exact-chain"):
        e["P2_EXACT"] = "1"
        if mode == "exact-chain":
            e["P2H_EXACT_CHAIN"] = "1"
    else:
        e["P2_GEMM"] = mode
    return e


def encdump(variant, mode, model_dir, wav, out_path, timeout=300):
    """(encoder frames [T, 640] fp32, token ids) of encdump_<variant> in the given GEMM mode."""
    r = subprocess.run([binary(f"encdump_{variant}"), model_dir, wav, out_path], env=env_for(mode),
                       capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"encdump_{variant} ({mode}) failed:\n{r.stdout}\n{r.stderr}"
    lines = r.stdout.strip().split("\n")
    T = int(lines[0].split()[1])
    ids = [int(x) for x in lines[1].split()] if len(lines) > 1 and lines[1].strip() else []
    frames = np.fromfile(out_path, dtype=np.float32)
    assert frames.size == T * JOINT, (frames.size, T)
    return frames.reshape(T, JOINT), ids


def cli_tokens(variant, mode, model_dir, wavs, timeout=300):
    """Token ids per file from the reference CLI (main.c --tokens) linked as phonon2_<variant>."""
    r = subprocess.run([binary(f"phonon2_{variant}"), "--tokens", model_dir, *wavs], env=env_for(mode),
                       capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"phonon2_{variant} ({mode}) failed:\n{r.stdout}\n{r.stderr}"
    out = {}
    for line in r.stdout.strip().split("\n"):
        path, _, ids = line.partition(": ")
        out[path] = [int(x) for x in ids.split()]
    assert len(out) == len(wavs), r.stdout
    return out
