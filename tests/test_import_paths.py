"""The reference's own import lines work unchanged against this package.

A caller of the reference writes ``import vkwr`` (reference vkwr/__init__.py:1-3),
``from vkwr._ops import import_all_ops`` (vkwr/_ops/__init__.py:1-5) and the
wrappers' ``from vkwr import _v1_wkv_C`` (vkwr/_ops/v1/v1_wkv_ops.py:3,
vkwr/_ops/rwkv7_ops.py:3).  Each runs here in a fresh interpreter, so no earlier
import in the test session can mask a failure.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Every op namespace the reference registers, with one op each that must be present after the import.
NAMESPACES = {
    "vkwr_v1_wkv": "wkv_forward_fp32",
    "vkwr_v1_linear": "linear_f16",
    "vkwr_v1_rank": "linear_wag_rank_in_f16",
    "vkwr_v1_mix": "tmix_mix6",
    "vkwr_v1_norm": "add_layer_norm_tmix_mix6_f16",
    "vkwr_rwkv7": "forward_seq",
    "vkwr_sampling": "temperature_topk_topp",
}


def _run(code):
    p = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-4000:] + p.stderr[-4000:]
    return p.stdout


def _probe(ns_ops):
    return "".join(f"assert hasattr(torch.ops.{ns}, {op!r}), {ns!r}\n" for ns, op in ns_ops.items())


def test_import_vkwr_registers_every_namespace():
    """reference vkwr/__init__.py:1-3: a bare `import vkwr` registers every op."""
    _run("import torch\nimport vkwr\n" + _probe(NAMESPACES) + "print('ok')\n")


def test_reference_package_lines_verbatim():
    """The reference's lines, as written there, in a fresh process: vkwr/__init__.py:1-3 and
    vkwr/_ops/__init__.py:1-5 (the module the latter imports, sampling_ops, is shipped here)."""
    code = (
        "import torch\n"
        "from vkwr._ops import import_all_ops\n"
        "\n"
        "import_all_ops()\n"
        "from vkwr._ops import rwkv7_ops, sampling_ops\n"
        "from vkwr._ops.v1 import import_all_v1_ops\n"
        "\n"
        "import_all_v1_ops()\n"
        + _probe(NAMESPACES)
    )
    _run(code)


@pytest.mark.parametrize("mod", ["_v1_wkv_C", "_v1_linear_C", "_v1_rank_C", "_v1_mix_C", "_v1_norm_C", "_rwkv7_C"])
def test_extension_module_lines_verbatim(mod):
    """The wrappers' `from vkwr import _v1_*_C` (e.g. vkwr/_ops/v1/v1_wkv_ops.py:3): the
    extension module itself is importable and registers its namespace."""
    ns = {"_v1_wkv_C": "vkwr_v1_wkv", "_v1_linear_C": "vkwr_v1_linear", "_v1_rank_C": "vkwr_v1_rank",
          "_v1_mix_C": "vkwr_v1_mix", "_v1_norm_C": "vkwr_v1_norm", "_rwkv7_C": "vkwr_rwkv7"}[mod]
    out = _run(f"import torch\nfrom vkwr import {mod}\nprint({mod}.__file__)\n" + _probe({ns: NAMESPACES[ns]}))
    assert os.path.dirname(out.strip().splitlines()[0]) == os.path.join(ROOT, "vkwr")


def test_reference_wrapper_modules_import_in_any_order():
    """Importing the wrapper modules directly (as reference callers do, e.g.
    `from vkwr._ops.v1 import v1_wkv_ops`) before or after `import vkwr` registers
    each fake implementation once (a second registration would raise)."""
    _run("import torch\nfrom vkwr._ops.v1 import v1_wkv_ops, v1_linear_ops\nimport vkwr\n"
         "from vkwr._ops import rwkv7_ops\nimport vkwr._ops.v1.v1_mix_ops\n" + _probe(NAMESPACES))


def test_model_executor_is_under_vkwr():
    """north_star: vkwr/model_executor calls the new ops; the decode driver lives there."""
    _run("import torch\nfrom vkwr.model_executor import DecodeEngine, MixedEngine, ContinuousBatcher\n")


@pytest.mark.gpu
def test_wkv_call_through_reference_import_paths(gpu):
    """One GPU call through the reference's import path and wrapper, checked bit-exact
    against the CPU oracle (config-0 distributions, B=1, T=3, H=2)."""
    import torch
    from vkwr._ops.v1 import v1_wkv_ops

    from oracle import oracle as orc
    from tests.wkv_inputs import make_state, make_wkv_inputs

    B, T, H = 1, 3, 2
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=7)
    S0 = make_state(B, H, seed=7, std=0.1)
    S_ref = S0.copy()
    y_ref = orc.wkv_fp32(B, T, C, H, S_ref, *ins, order="seq")
    st = torch.from_numpy(S0).to(gpu)
    y = v1_wkv_ops.wkv_forward_seq_fp32(B, T, C, H, st, *(torch.from_numpy(x).to(gpu) for x in ins))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), y_ref.view(np.uint16))
    assert np.array_equal(st.cpu().numpy(), S_ref)
