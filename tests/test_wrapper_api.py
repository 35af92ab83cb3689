"""The host interface mirrors the reference's wrapper module (wrapper.py:7-212): the same
public names, and the hooks FAIRChem's predict unit calls behave as the reference's do
(no GPU needed)."""
import types

import pytest


def test_module_names_match_reference():
    import wrapper
    for name in ("ZeroAllocBackbone", "transfer_weights", "validate_atoms_data", "on_predict_check",
                 "prepare_for_inference"):
        assert callable(getattr(wrapper, name)), name
    for name in ("validate_atoms_data", "on_predict_check", "prepare_for_inference", "csd_embedding", "forward"):
        assert callable(getattr(wrapper.ZeroAllocBackbone, name)), name


@pytest.mark.parametrize("task,spin", [("omol", 1), ("omat", 0), ("oc20", 0)])
def test_validate_atoms_data_defaults(task, spin):
    """Missing charge and spin default to 0 and (1 for omol, else 0); given values stay."""
    import wrapper
    atoms = types.SimpleNamespace(info={})
    for fn in (wrapper.validate_atoms_data, wrapper.ZeroAllocBackbone.validate_atoms_data):
        atoms.info = {}
        fn(None, atoms, task)
        assert atoms.info == {"charge": 0, "spin": spin}
        atoms.info = {"charge": -2, "spin": 3}
        fn(None, atoms, task)
        assert atoms.info == {"charge": -2, "spin": 3}


def test_prepare_for_inference_returns_self_and_check_is_bypassed():
    import wrapper
    obj = object()
    assert wrapper.prepare_for_inference(obj, None, None) is obj
    assert wrapper.on_predict_check(obj, None) is None
