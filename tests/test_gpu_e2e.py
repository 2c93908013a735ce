"""End to end on the GPU: the reference engine (built from its own sources, oracle/Makefile) with its quantised
GEMMs bound to libphonon2_gemm.so, against the same engine with its own GEMMs (exact mode) and with the oracle's
(int8w, int8), on a synthetic model in the reference's weights.bin format.

The encoder frames – the output of all 24 blocks' 216 five-value linears, the int8 subsampling and projector
linears and everything between them – must be bit-identical (exact mode on the fmaf-chain route, P2H_EXACT_CHAIN=1,
and the int8 modes), and the greedy TDT decoder must emit the same token ids; the reference CLI (main.c --tokens,
through p2_engine_open / p2_transcribe) must print the same ids. Exact mode on the fp32 matrix cores sums in another
order: its frames agree to fp32 rounding and its token ids are identical."""
import numpy as np
import pytest

from e2e import model, run

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not run.have("encdump_cpu", "encdump_gpu", "encdump_oracle", "phonon2_cpu",
                                              "phonon2_gpu", "phonon2_oracle"),
                                 reason="oracle/_ref engines not built")]


@pytest.fixture(scope="module")
def fx(tmp_path_factory):
    d = tmp_path_factory.mktemp("e2e_gpu")
    print(f"writing the synthetic model under {d}", flush=True)
    model.write_model(str(d / "model"))
    model.write_wav(str(d / "a.wav"), 3.0, seed=5)
    model.write_wav(str(d / "b.wav"), 1.5, seed=11)
    return str(d)


@pytest.mark.parametrize("mode,reference", [("exact-chain", "cpu"), ("int8w", "oracle"), ("int8", "oracle")])
def test_encoder_frames_and_tokens(fx, mode, reference):
    print(f"encdump_gpu vs encdump_{reference}, {mode}", flush=True)
    got, got_ids = run.encdump("gpu", mode, fx + "/model", fx + "/a.wav", fx + f"/gpu_{mode}.f32")
    ref, ref_ids = run.encdump(reference, mode, fx + "/model", fx + "/a.wav", fx + f"/{reference}_{mode}.f32")
    neq = got.view(np.uint32) != ref.view(np.uint32)
    assert not neq.any(), f"{neq.sum()} of {neq.size} encoder values differ; first at {np.argwhere(neq)[0]}"
    assert got_ids == ref_ids
    assert len(ref_ids) >= 8 and len(set(ref_ids)) >= 5, ref_ids


def test_encoder_exact_on_matrix_cores(fx):
    """Exact mode on the fp32 matrix cores: the products are summed in another order than the reference's fmaf
    chain, so frames agree to fp32 rounding carried through 24 blocks, and the token ids are identical."""
    print("encdump_gpu (exact, matrix cores) vs encdump_cpu", flush=True)
    got, got_ids = run.encdump("gpu", "exact", fx + "/model", fx + "/a.wav", fx + "/gpu_exact_mfma.f32")
    ref, ref_ids = run.encdump("cpu", "exact", fx + "/model", fx + "/a.wav", fx + "/cpu_exact.f32")
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    err = np.max(np.abs(got.astype(np.float64) - ref)) / rms
    print(f"max |gpu - cpu| / rms(frames) = {err:.3g}", flush=True)
    assert err < 1e-3
    assert got_ids == ref_ids


@pytest.mark.skipif(not run.have("encdump_gpuall"), reason="oracle/_ref/encdump_gpuall not built")
@pytest.mark.parametrize("mode,reference", [("exact-chain", "cpu"), ("int8w", "oracle")])
def test_encoder_every_gemm_on_gpu(fx, mode, reference):
    """The engine with no blas.c at all: every blas.h function from the GPU library, so the fp32 GEMMs of attention
    (p2_sgemm_st per head, encoder.c:279-316) and of the subsampling run on the matrix cores as well. They sum in
    another order than the reference's CPU sgemm, so the frames agree to fp32 rounding carried through 24 blocks
    (against the same mode with the CPU's fp32 GEMMs) and the token ids are identical."""
    print(f"encdump_gpuall vs encdump_{reference}, {mode}", flush=True)
    got, got_ids = run.encdump("gpuall", mode, fx + "/model", fx + "/a.wav", fx + f"/gpuall_{mode}.f32")
    ref, ref_ids = run.encdump(reference, mode, fx + "/model", fx + "/a.wav", fx + f"/{reference}_{mode}_all.f32")
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    err = np.max(np.abs(got.astype(np.float64) - ref)) / rms
    print(f"max |gpu - ref| / rms(frames) = {err:.3g}", flush=True)
    assert err < 1e-3
    assert got_ids == ref_ids


@pytest.mark.parametrize("mode,reference", [("exact-chain", "cpu"), ("exact", "cpu"), ("int8w", "oracle")])
def test_cli_token_ids(fx, mode, reference):
    wavs = [fx + "/a.wav", fx + "/b.wav"]
    print(f"phonon2_gpu vs phonon2_{reference}, {mode}", flush=True)
    got = run.cli_tokens("gpu", mode, fx + "/model", wavs)
    ref = run.cli_tokens(reference, mode, fx + "/model", wavs)
    assert got == ref
    assert all(len(v) > 0 for v in ref.values())
