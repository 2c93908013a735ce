"""The synthetic model and audio of the end-to-end tests, checked on the CPU with the reference engine as it ships
(oracle/_ref/encdump_cpu, exact mode) and with its quantised GEMMs on the oracle (encdump_oracle, int8w): the files
load through the reference's strict loader, the encoder frames vary with the audio, the greedy decoder emits a
varied token stream, and the int8w frames stay within the quantisation error of the exact ones."""
import os

import numpy as np
import pytest

from e2e import model, run

pytestmark = pytest.mark.skipif(not run.have("encdump_cpu", "encdump_oracle"),
                                reason="oracle/_ref engines not built (oracle/Makefile needs the reference tree)")


@pytest.fixture(scope="module")
def fixture_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("e2e")
    model.write_model(str(d / "model"))
    model.write_wav(str(d / "a.wav"), 3.0, seed=5)
    return d


def test_reference_engine_decodes_the_synthetic_model(fixture_dir):
    d = str(fixture_dir)
    frames, ids = run.encdump("cpu", "exact", d + "/model", d + "/a.wav", d + "/cpu.f32")
    assert frames.shape == (38, run.JOINT)   # 3 s: 300 mel frames, three stride-2 convolutions
    assert np.isfinite(frames).all()
    assert frames.std(axis=0).mean() > 0.3 * frames.mean(axis=0).std(), "frames must vary with the audio"
    assert len(ids) >= 8 and len(set(ids)) >= 5, ids


def test_oracle_engine_int8w_within_quantisation_error(fixture_dir):
    d = str(fixture_dir)
    exact, _ = run.encdump("cpu", "exact", d + "/model", d + "/a.wav", d + "/cpu.f32")
    q, ids = run.encdump("oracle", "int8w", d + "/model", d + "/a.wav", d + "/oracle.f32")
    rel = np.abs(q - exact).max() / np.abs(exact).max()
    assert 0 < rel < 0.15, rel
    assert len(ids) >= 8
