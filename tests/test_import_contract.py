"""The missing-library contract of the drop-in boundary (CPU, no GPU needed).

The reference imports every kernel module inside ``try/except Exception`` and, on
failure, sets the op to ``None`` and its flag to False, then takes its eager path
(``inference/models/atma.py:31-80``).  Here the ops package raises ``ImportError``
when libatma_hip.so cannot be loaded, so that guard works unchanged when the reference's
kernel imports are pointed at the ``atma_amd.kernel`` modules of the same names; with the
library present, every reference-named module exports the reference's names and flag."""

import subprocess
import sys
import textwrap
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

# The reference's guarded imports (inference/models/atma.py:31-80), with the module
# paths swapped to this package's reference-named modules.
GUARDED = textwrap.dedent("""
    try:
        from atma_amd.kernel.polar_triton import (polar_attention_fwd, polar_attention_packed_fwd,
                                                  polar_attention_decode, HAS_TRITON)
    except Exception:
        polar_attention_fwd = None
        polar_attention_packed_fwd = None
        polar_attention_decode = None
        HAS_TRITON = False
    try:
        from atma_amd.kernel.gated_delta_triton import chunk_gated_delta_rule
        _HAS_FLA = True
    except Exception:
        chunk_gated_delta_rule = None
        _HAS_FLA = False
    try:
        from atma_amd.kernel.gated_delta_triton import gated_delta_decode_step
        from atma_amd.kernel.gated_delta_triton import HAS_TRITON as _HAS_STEP_KERNEL
    except Exception:
        gated_delta_decode_step = None
        _HAS_STEP_KERNEL = False
    try:
        from atma_amd.kernel.causal_conv1d_triton import causal_conv1d_decode_step
        from atma_amd.kernel.causal_conv1d_triton import HAS_TRITON as _HAS_CONV_STEP_KERNEL
    except Exception:
        causal_conv1d_decode_step = None
        _HAS_CONV_STEP_KERNEL = False
    try:
        from atma_amd.kernel.inference_ops_triton import squared_relu_gate, softcap_logits, packed_causal_conv1d
        from atma_amd.kernel.inference_ops_triton import HAS_TRITON as _HAS_INFERENCE_OPS
    except Exception:
        squared_relu_gate = None
        softcap_logits = None
        packed_causal_conv1d = None
        _HAS_INFERENCE_OPS = False
    ops = [polar_attention_fwd, polar_attention_packed_fwd, polar_attention_decode,
           chunk_gated_delta_rule, gated_delta_decode_step, causal_conv1d_decode_step,
           squared_relu_gate, softcap_logits, packed_causal_conv1d]
    flags = [HAS_TRITON, _HAS_FLA, _HAS_STEP_KERNEL, _HAS_CONV_STEP_KERNEL, _HAS_INFERENCE_OPS]
""")


def _run(prelude):
    code = prelude + GUARDED + textwrap.dedent("""
        print("OPS", sum(o is not None for o in ops), len(ops))
        print("FLAGS", [bool(f) for f in flags])
    """)
    proc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 0, proc.stderr
    return proc.stdout


def test_missing_library_takes_the_reference_fallback():
    out = _run(textwrap.dedent("""
        from pathlib import Path
        import atma_amd._lib as L
        L.LIB_PATH = Path("/nonexistent/libatma_hip.so")   # the library is not there
        try:
            import atma_amd.kernel
            raise SystemExit("atma_amd.kernel imported without its library")
        except ImportError as e:
            assert isinstance(e, L.HipLibraryMissing) and isinstance(e, RuntimeError), type(e)
    """))
    assert "OPS 0 9" in out, out
    # only FLA's flag is set by the import guard itself, and it too stays False
    assert "FLAGS [False, False, False, False, False]" in out, out


def test_present_library_exports_reference_names():
    if not (ROOT / "atma_amd" / "libatma_hip.so").exists():
        import pytest
        pytest.fail("libatma_hip.so missing: run `python -m atma_amd._build`")
    out = _run("")
    assert "OPS 9 9" in out, out
    # the ops import; HAS_TRITON follows GPU visibility (False on a CPU-only host)
    import torch
    gpu = torch.cuda.is_available()
    assert f"FLAGS [{gpu}, True, {gpu}, {gpu}, {gpu}]" in out, out
