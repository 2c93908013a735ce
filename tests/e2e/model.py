"""A synthetic Phonon-2 model in the reference engine's on-disk format, and synthetic audio, for end-to-end tests.

Writes weights.bin, weights.json and tokens.txt the way the reference's converter lays them out
(convert_weights.py:83-125, 160-225): every tensor 64-byte aligned; "float32" entries with offset/shape/numel;
"int8" tables with one fp32 scale per output feature (per column for GEMM tables [in, out], per row for decoder
tables [out, in]); "five_value" entries with the 2-bit sign plane [K][N/4] (code = sign + 1 at bits 2·(n % 4)) and the
little-endian hi-flag plane [K][N/8]; a "_meta" entry with the format name the loader checks (weights.c:420-427). The
tensor names and shapes are the ones the loader looks up (weights.c:433-511).

The values are random (seeded): five-value columns with lo ~ U(0.005, 0.02) and hi = lo·U(2, 4), both rounded to
fp16 values, codes 0 / ±lo / ±hi with probabilities 0.4 / 0.4 / 0.2; int8 tables with 6-bit codes; norms near 1.
"""
import json
import os
import wave

import numpy as np

ALIGN = 64
FORMAT = "phonon-2-c-weights-v1"
D, FF, C, H, E, J = 1024, 4096, 256, 640, 640, 640
N_BLOCKS, VOCAB, N_LOGITS, N_MELS, SUB = 24, 8193, 8198, 128, 8


class _Container:
    """The tensors of weights.bin and the manifest that locates them. Tensors are laid out first (each at the next
    ALIGN boundary, the gaps zero) and written in one pass by save(); manifest entries carry the format's field
    names (weights.c:433-511), so the reference's loader reads them unchanged."""

    def __init__(self):
        self.parts = []        # (offset, contiguous array) in file order
        self.end = 0
        self.manifest = {}

    def _place(self, arr, dtype):
        arr = np.ascontiguousarray(arr, dtype=dtype)
        at = (self.end + ALIGN - 1) // ALIGN * ALIGN
        self.parts.append((at, arr))
        self.end = at + arr.nbytes
        return at

    def tensor(self, name, kind, shape, fields=(), **extra):
        """One manifest entry: `fields` are (key, array, dtype) triples, each array placed and its offset stored."""
        entry = {"dtype": kind, "shape": [int(d) for d in shape], **extra}
        for key, arr, dtype in fields:
            entry[key] = self._place(arr, dtype)
        self.manifest[name] = entry

    def f32(self, name, arr):
        arr = np.asarray(arr, np.float32)
        self.tensor(name, "float32", arr.shape, [("offset", arr, np.float32)], numel=int(arr.size))

    def i8(self, name, q, scales):
        self.tensor(name, "int8", q.shape, [("offset", q, np.int8), ("scales_offset", scales, np.float32)])

    def fv(self, name, signs, flags, lo, hi, K, N):
        self.tensor(name, "five_value", (K, N), [("signs_offset", signs, np.uint8), ("flags_offset", flags, np.uint8),
                                                 ("lo_offset", lo, np.float32), ("hi_offset", hi, np.float32)])

    def save(self, path):
        with open(path, "wb") as f:
            for at, arr in self.parts:
                f.write(b"\0" * (at - f.tell()))
                f.write(arr.tobytes())


def _fp16(x):
    return x.astype(np.float16).astype(np.float32)


def five_value(rng, K, N, scale=1.0):
    """Packed planes and fp16-valued lo/hi of one random five-value weight [K, N]."""
    r = rng.integers(0, 10, size=(K, N), dtype=np.uint8)
    code = np.where(r < 4, 1, np.where(r & 1, 0, 2)).astype(np.uint8)   # 0: −1, 1: 0, 2: +1
    is_hi = r >= 8
    c4 = code.reshape(K, N // 4, 4)
    signs = (c4[..., 0] | (c4[..., 1] << 2) | (c4[..., 2] << 4) | (c4[..., 3] << 6)).astype(np.uint8)
    flags = np.packbits(is_hi, axis=1, bitorder="little")
    lo = _fp16(scale * rng.uniform(0.005, 0.02, N).astype(np.float32))
    hi = _fp16(lo * rng.uniform(2.0, 4.0, N).astype(np.float32))
    return signs, flags, lo, hi


def _i8(rng, rows, cols, per_row, gain):
    q = rng.integers(-31, 32, size=(rows, cols), dtype=np.int8)
    fan_in = cols if per_row else rows
    scales = np.full(rows if per_row else cols, gain / (18.0 * np.sqrt(fan_in)), np.float32)
    scales *= rng.uniform(0.8, 1.25, scales.shape).astype(np.float32)
    return q, scales


def write_model(out_dir, seed=7, bias=0.0, joint_gain=3.0, attn_scale=0.05):
    """Write weights.bin, weights.json and tokens.txt into out_dir (about 250 MB). `bias` scales every bias and
    LayerNorm offset (0 keeps the encoder frames a function of the audio alone); `attn_scale` scales the attention
    output projection (random attention is close to uniform, and its frame average would otherwise swamp the
    frame-to-frame variation the decoder sees)."""
    os.makedirs(out_dir, exist_ok=True)
    rng = np.random.default_rng(seed)
    w = _Container()
    n = lambda *shape, s=1.0: (rng.standard_normal(shape) * s).astype(np.float32)
    for layer in (0, 2, 5):
        w.f32(f"subsampling.conv.{layer}.weight", n(C, 9, s=0.3))
        w.f32(f"subsampling.conv.{layer}.bias", n(C, s=0.05 * bias))
    for layer in (3, 6):
        w.f32(f"subsampling.conv.{layer}.weight", n(C, C, s=1.0 / 16))
        w.f32(f"subsampling.conv.{layer}.bias", n(C, s=0.05 * bias))
    w.i8("subsampling.linear.weight", *_i8(rng, C * (N_MELS // SUB), D, False, 1.0))
    w.f32("subsampling.linear.bias", n(D, s=0.05 * bias))
    for i in range(N_BLOCKS):
        o = f"layers.{i}"
        for norm in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
            w.f32(f"{o}.{norm}.weight", 1.0 + n(D, s=0.1))
            w.f32(f"{o}.{norm}.bias", n(D, s=0.1 * bias))
        for name, K, N in ((f"{o}.feed_forward1.linear1.weight", D, FF), (f"{o}.feed_forward1.linear2.weight", FF, D),
                           (f"{o}.feed_forward2.linear1.weight", D, FF), (f"{o}.feed_forward2.linear2.weight", FF, D),
                           (f"{o}.self_attn.qkv_proj.weight", D, 3 * D), (f"{o}.self_attn.relative_k_proj.weight", D, D),
                           (f"{o}.self_attn.o_proj.weight", D, D), (f"{o}.conv.pointwise_conv1.weight", D, 2 * D),
                           (f"{o}.conv.pointwise_conv2.weight", D, D)):
            w.fv(name, *five_value(rng, K, N, attn_scale if "o_proj" in name else 1.0), K, N)
        w.f32(f"{o}.self_attn.bias_u", n(D, s=0.1))
        w.f32(f"{o}.self_attn.bias_v", n(D, s=0.1))
        w.f32(f"{o}.conv.depthwise_conv.weight", n(D, 9, s=0.3))
        w.f32(f"{o}.conv.depthwise_conv.bias", n(D, s=0.05 * bias))
    w.i8("encoder_projector.weight", *_i8(rng, D, J, False, 1.0))
    w.f32("encoder_projector.bias", n(J, s=0.05 * bias))
    q, s = _i8(rng, VOCAB, E, True, 1.0)
    q[VOCAB - 1] = 0   # the blank row (convert_weights.py:207)
    w.i8("decoder.embedding.weight", q, s)
    for layer in range(2):
        w.i8(f"decoder.lstm.weight_ih_l{layer}", *_i8(rng, 4 * H, E if layer == 0 else H, True, 1.0))
        w.i8(f"decoder.lstm.weight_hh_l{layer}", *_i8(rng, 4 * H, H, True, 1.0))
        w.f32(f"decoder.lstm.bias_ih_l{layer}", n(4 * H, s=0.1))
        w.f32(f"decoder.lstm.bias_hh_l{layer}", n(4 * H, s=0.1))
    w.i8("decoder.decoder_projector.weight", *_i8(rng, J, H, True, 1.0))
    w.f32("decoder.decoder_projector.bias", n(J, s=0.05))
    w.i8("joint.head.weight", *_i8(rng, N_LOGITS, J, True, joint_gain))
    w.f32("joint.head.bias", n(N_LOGITS, s=0.1))
    w.save(os.path.join(out_dir, "weights.bin"))
    w.manifest["_meta"] = {"format": FORMAT, "converter": "tests/e2e/model.py (synthetic)"}
    with open(os.path.join(out_dir, "weights.json"), "w") as f:
        json.dump(w.manifest, f, indent=1)
        f.write("\n")
    with open(os.path.join(out_dir, "tokens.txt"), "w", encoding="utf-8") as f:
        f.write("\n".join([f"▁t{i}" for i in range(VOCAB - 1)] + ["<blank>"]) + "\n")
    return out_dir


def write_wav(path, seconds=2.0, seed=3, rate=16000):
    """Mono 16-bit PCM: a few gliding harmonic tones under syllable-rate envelopes, plus noise."""
    rng = np.random.default_rng(seed)
    t = np.arange(int(seconds * rate)) / rate
    x = np.zeros_like(t)
    for f0 in rng.uniform(110, 260, 3):
        glide = f0 * (1 + 0.15 * np.sin(2 * np.pi * rng.uniform(0.5, 2.0) * t))
        phase = 2 * np.pi * np.cumsum(glide) / rate
        env = 0.5 * (1 + np.sin(2 * np.pi * rng.uniform(3, 6) * t + rng.uniform(0, 6.28)))
        for h in range(1, 6):
            x += env * np.sin(h * phase) / h
    x += 0.05 * rng.standard_normal(t.size)
    pcm = np.clip(x / np.max(np.abs(x)) * 0.6 * 32767, -32768, 32767).astype("<i2")
    with wave.open(path, "wb") as wf:
        wf.setnchannels(1)
        wf.setsampwidth(2)
        wf.setframerate(rate)
        wf.writeframes(pcm.tobytes())
    return path
