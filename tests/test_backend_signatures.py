"""The decode entries' signatures against the backend's gfx950 call sites (no GPU needed).

``reference/turboquant_attn.py`` calls ``flydsl_turboquant_decode_attention`` with the kwargs
of ``:1161-1183`` and ``_dispatch_decode_soa`` with those of ``:1194-1216``; the latter keeps
only the kwargs its target's signature names and raises ``NotImplementedError`` for any other
non-None one (``:1241-1257``).  The parameter lists below are those of
``reference/flydsl_decode.py:559-581`` and ``reference/soa_unified.py:1291-1313``, in order.
"""
import inspect

import pytest

from tq4_decode import flydsl_decode, soa_decode, soa_unified

BACKEND_SOA_KWARGS = (
    "query", "kv_cache", "block_table", "seq_lens", "Pi", "centroids", "scale", "mse_bits",
    "key_packed_size", "value_quant_bits", "value_packed_size", "max_seq_len", "key_fp8",
    "norm_correction", "PiT", "mid_o_buf", "output_buf", "lse_buf", "buf_holder",
    "max_num_kv_splits", "sinks", "sliding_window")
BACKEND_FLYDSL_KWARGS = tuple(k for k in BACKEND_SOA_KWARGS if k != "sliding_window")

REFERENCE_PARAMS = (
    "query", "kv_cache", "block_table", "seq_lens", "Pi", "centroids", "scale", "mse_bits",
    "key_packed_size", "value_quant_bits", "value_packed_size", "key_fp8", "norm_correction", "PiT",
    "max_seq_len", "mid_o_buf", "output_buf", "lse_buf", "buf_holder", "max_num_kv_splits", "sinks")
REFERENCE_DEFAULTS = {"key_fp8": False, "norm_correction": False, "PiT": None, "max_seq_len": 0,
                      "mid_o_buf": None, "output_buf": None, "lse_buf": None, "buf_holder": None,
                      "max_num_kv_splits": 32, "sinks": None}


def _filter(fn, kwargs):
    """The signature filter of ``_dispatch_decode_soa``; returns the kwargs it passes on."""
    accepted = set(inspect.signature(fn).parameters)
    dropped = [k for k, v in kwargs.items() if k not in accepted and v is not None]
    if dropped:
        raise NotImplementedError(f"SoA decode does not support kwargs {sorted(dropped)}")
    return {k: v for k, v in kwargs.items() if k in accepted}


@pytest.mark.parametrize("fn", [soa_unified.triton_turboquant_decode_attention_soa,
                                flydsl_decode.flydsl_turboquant_decode_attention])
def test_parameters_are_the_references(fn):
    params = inspect.signature(fn).parameters
    assert tuple(params) == REFERENCE_PARAMS
    for name, default in REFERENCE_DEFAULTS.items():
        assert params[name].default == default, name
    for name in REFERENCE_PARAMS[:11]:
        assert params[name].default is inspect.Parameter.empty, name


def test_backend_soa_call_passes_the_filter():
    kwargs = {k: object() for k in BACKEND_SOA_KWARGS}
    kwargs["sliding_window"] = None  # a layer without a window
    passed = _filter(soa_unified.triton_turboquant_decode_attention_soa, kwargs)
    assert set(passed) == set(BACKEND_SOA_KWARGS) - {"sliding_window"}
    # a layer with a window raises, as with the reference adapter (no such parameter)
    with pytest.raises(NotImplementedError, match="sliding_window"):
        _filter(soa_unified.triton_turboquant_decode_attention_soa, {**kwargs, "sliding_window": 4096})


def test_backend_soa_call_is_refused_by_the_v1_signature():
    """The v1 entry (``reference/soa_decode_v1.py:485-506``) takes neither value_packed_size nor
    max_seq_len: the backend cannot route its gfx950 calls there."""
    kwargs = {k: object() for k in BACKEND_SOA_KWARGS}
    kwargs["sliding_window"] = None
    with pytest.raises(NotImplementedError, match="max_seq_len"):
        _filter(soa_decode.triton_turboquant_decode_attention.func, kwargs)


def test_backend_flydsl_call_binds():
    sig = inspect.signature(flydsl_decode.flydsl_turboquant_decode_attention)
    sig.bind(**{k: object() for k in BACKEND_FLYDSL_KWARGS})


def test_flydsl_entry_checks_the_preset():
    """The reference's asserts (``reference/flydsl_decode.py:604-608``) fire before any tensor
    is touched."""
    f = flydsl_decode.flydsl_turboquant_decode_attention
    base = dict(query=None, kv_cache=None, block_table=None, seq_lens=None, Pi=None, centroids=None,
                scale=1.0, mse_bits=4, key_packed_size=66, value_quant_bits=4, value_packed_size=68)
    with pytest.raises(AssertionError, match="MSE-key"):
        f(**{**base, "key_fp8": True})
    with pytest.raises(AssertionError, match="mse_bits=4"):
        f(**{**base, "mse_bits": 3})
    with pytest.raises(AssertionError, match="value_quant_bits=4"):
        f(**{**base, "value_quant_bits": 3})


def test_soa_adapter_value_packed_size():
    assert soa_unified.value_packed_bytes(128, 4) == 68
    assert soa_unified.value_packed_bytes(128, 3) == 52
