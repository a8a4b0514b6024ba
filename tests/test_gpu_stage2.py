"""Stage2 and full-decode parity on the GPU."""
import numpy as np
import pytest
import torch

from conftest import to_dev
from oracle import native, stage1 as ostage
from tq4_decode import ops, workloads

pytestmark = pytest.mark.gpu


def _mid_on_gpu(w, dev):
    mid = torch.full((w.batch, w.num_q_heads, w.num_kv_splits, 129), float("nan"), device=dev)
    ops.stage1(to_dev(w.q_rot, dev), to_dev(w.kv_cache, dev), to_dev(w.block_table, dev),
               to_dev(w.seq_lens, dev), to_dev(w.pair_lut, dev), mid)
    return mid


@pytest.mark.parametrize("lens,splits", [([1, 3, 17, 100, 257, 999], 32), ([4096, 4095], 32),
                                         ([5000, 70], 64), ([64], 1), ([9999, 5000, 33], 100)])
def test_stage2_matches_oracle_and_skips_empty_splits(dev, lens, splits):
    w = workloads.small(201, len(lens), lens, splits)
    mid = _mid_on_gpu(w, dev)  # empty splits hold NaN: merging one would poison the output
    out, lse = ops.stage2(mid, to_dev(w.seq_lens, dev))
    torch.cuda.synchronize()
    ro, rl = native.stage2(mid.cpu().numpy(), w.seq_lens)
    assert np.isfinite(out.cpu().numpy()).all()
    assert np.abs(out.cpu().numpy() - ro).max() <= 1e-5
    assert np.abs(lse.cpu().numpy() - rl).max() <= 1e-5
    fo, fl = ostage.attention_reference(w.q_rot, w.kv_cache, w.block_table, w.seq_lens,
                                        w.centroids, num_kv_heads=8)
    assert np.abs(out.cpu().numpy() - fo).max() <= 1e-4
    assert np.abs(lse.cpu().numpy() - fl).max() <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_stage2_output_dtypes(dev, dtype):
    w = workloads.small(202, 3, [300, 45, 1000], 16)
    mid = _mid_on_gpu(w, dev)
    ref, _ = ops.stage2(mid, to_dev(w.seq_lens, dev))
    got, _ = ops.stage2(mid, to_dev(w.seq_lens, dev), out_dtype=dtype)
    assert torch.equal(got, ref.to(dtype))


def test_reference_stage2_call_shapes(dev):
    w = workloads.small(203, 2, [4096, 4096], 32)
    sl = to_dev(w.seq_lens, dev)
    mid = _mid_on_gpu(w, dev)
    out = torch.empty(2, 32, 128, device=dev)
    lse = torch.empty(2, 32, device=dev)
    ops.launch_stage2(mid, sl, out, lse)
    out7 = torch.empty_like(out)
    lse7 = torch.empty_like(lse)
    ops.ext.tq4_cuda_v7_stage2(mid, out7, lse7, sl)
    torch.cuda.synchronize()
    assert torch.equal(out, out7) and torch.equal(lse, lse7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows", [1, 64, 65, 120, 8192])
def test_rotate_query_matches_fp64(dev, dtype, rows):
    """Matrix-core rotation (f16 hi/lo splits) vs an fp64 matmul of the same inputs;
    row counts around the 64-row workgroup tile."""
    rng = np.random.default_rng(204)
    q = torch.from_numpy(rng.standard_normal((rows, 128)).astype(np.float32)).to(dtype)
    rot = workloads.random_orthogonal(rng, 128)
    got = ops.rotate_query(q.to(dev), to_dev(rot, dev)).cpu().numpy()
    ref = q.double().numpy() @ rot.astype(np.float64)
    err = np.abs(got - ref).max()
    print(f"rotation max-abs {err:.3e}")
    assert err <= 2e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_rotate_query_rows_of_any_magnitude(dev, dtype):
    """Rows whose magnitudes lie far outside the f16 range (bf16 / fp32 up to 1e30, down to
    1e-30) and rows mixing large and small elements: each row is scaled by a power of two
    before the f16 split, so the error relative to the row's norm stays at the fp32 level."""
    rng = np.random.default_rng(208)
    rows = 96
    x = rng.standard_normal((rows, 128))
    mags = {torch.bfloat16: [1e30, 1e12, 7e4, 1.0, 1e-6, 1e-20, 1e-30],
            torch.float32: [1e30, 1e12, 7e4, 1.0, 1e-6, 1e-20, 1e-30],
            torch.float16: [1e4, 1.0, 1e-3, 1e-5]}[dtype]
    x *= np.array(mags)[np.arange(rows) % len(mags)][:, None]
    x[rows - 1, :64] *= 1e-3  # a row with a 1000x spread
    x[rows - 2] = 0.0
    q = torch.from_numpy(x.astype(np.float32)).to(dtype)
    rot = workloads.random_orthogonal(rng, 128)
    got = ops.rotate_query(q.to(dev), to_dev(rot, dev)).cpu().numpy().astype(np.float64)
    ref = q.double().numpy() @ rot.astype(np.float64)
    assert np.isfinite(got).all()
    norm = np.maximum(np.linalg.norm(ref, axis=1, keepdims=True), 1e-300)
    rel = (np.abs(got - ref) / norm).max()
    print(f"{dtype} rotation error / row norm {rel:.3e}")
    assert rel <= 2e-6
    assert np.array_equal(got[rows - 2], np.zeros(128))


def test_full_b256_ctx2048_bf16(dev):
    w = workloads.full_b256_ctx2048()
    t = lambda a: to_dev(a, dev)  # noqa: E731
    out, lse = ops.full_decode(t(w.query), t(w.rotation_t), t(w.kv_cache), t(w.block_table),
                               t(w.seq_lens), t(w.centroids), w.num_kv_splits,
                               out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    q_rot = (w.query.astype(np.float64) @ w.rotation_t.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, w.kv_cache, w.block_table, w.seq_lens, w.centroids,
                        w.num_kv_splits, num_kv_heads=8)
    ro, rl = native.stage2(mid, w.seq_lens)
    err = np.abs(out.float().cpu().numpy() - ro).max()
    print(f"full decode bf16 max-abs {err:.3e}")
    assert err <= 1e-3
    assert np.abs(lse.cpu().numpy() - rl).max() <= 1e-4


def test_full_decode_reference_ext_shape(dev):
    w = workloads.small(205, 4, [4096, 2000, 1, 77], 32)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    mid = torch.empty(4, 32, 32, 129, device=dev)
    out = torch.empty(4, 32, 128, device=dev)
    lse = torch.empty(4, 32, device=dev)
    ops.ext.tq4_cuda_v7_full(t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens),
                             t(w.centroids), mid, out, lse)
    torch.cuda.synchronize()
    fo, fl = ostage.attention_reference(w.q_rot, w.kv_cache, w.block_table, w.seq_lens,
                                        w.centroids, num_kv_heads=8)
    assert np.abs(out.cpu().numpy() - fo).max() <= 1e-4
    assert np.abs(lse.cpu().numpy() - fl).max() <= 1e-4


def test_ext_stage2_without_seq_lens_merges_every_split(dev):
    """``ext.tq4_cuda_v7_stage2(mid_o, output, lse)`` has the reference V7 signature, without
    seq_lens (``cuda/tq4_cuda_v7.cu:56-76``), and merges every split of every row, as that
    kernel does: its precondition is that Stage1 wrote all of them, i.e. every length gives
    S non-empty splits (``ceil(len / ceil(len / S)) == S``: 77 tokens over 32 splits of 3
    leave 6 empty).  Lengths that are multiples of 32 over 32 splits: the result equals the
    merge of the non-empty splits (the seq_lens form) bit for bit, and the oracle."""
    w = workloads.small(206, 4, [4096, 2016, 32, 96], 32)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    mid = torch.full((4, 32, 32, 129), float("nan"), device=dev)
    ops.ext.tq4_cuda_v7_stage1(t(w.q_rot), t(w.kv_cache), t(w.block_table), t(w.seq_lens),
                               t(w.centroids), mid)
    out, lse = torch.empty(4, 32, 128, device=dev), torch.empty(4, 32, device=dev)
    ops.ext.tq4_cuda_v7_stage2(mid, out, lse)
    out2, lse2 = torch.empty_like(out), torch.empty_like(lse)
    ops.ext.tq4_cuda_v7_stage2(mid, out2, lse2, t(w.seq_lens))
    torch.cuda.synchronize()
    assert not torch.isnan(mid).any(), "every split was written"
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    fo, fl = ostage.attention_reference(w.q_rot, w.kv_cache, w.block_table, w.seq_lens,
                                        w.centroids, num_kv_heads=8)
    assert np.abs(out.cpu().numpy() - fo).max() <= 1e-4
    assert np.abs(lse.cpu().numpy() - fl).max() <= 1e-4


@pytest.mark.parametrize("layout", ["soa", "aos"])
def test_backend_decode_entry(dev, layout):
    """``tq4_decode.{soa,aos}_decode.triton_turboquant_decode_attention`` with the backend's
    arguments (Pi, not PiT; workspace buffers; fixed split count) against the oracle."""
    from tq4_decode import aos_decode, soa_decode

    rng = np.random.default_rng(206)
    w = workloads.small(206, 5, [1500, 1, 333, 4096, 64], 32)
    query = rng.standard_normal((5, 32, 128)).astype(np.float16)
    rot_t = workloads.random_orthogonal(rng, 128)
    cache = workloads.soa_to_aos(w.kv_cache, w.centroids, 8) if layout == "aos" else w.kv_cache
    t = lambda a: to_dev(a, dev)  # noqa: E731
    mid_buf = torch.empty(8, 32, 32, 129, device=dev)
    out_buf = torch.empty(8, 32, 128, dtype=torch.float16, device=dev)
    lse_buf = torch.empty(8, 32, device=dev)

    class Holder:
        pass

    mod = aos_decode if layout == "aos" else soa_decode
    out = mod.triton_turboquant_decode_attention(
        t(query), t(cache), t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids),
        128 ** -0.5, mse_bits=4, key_packed_size=66, value_quant_bits=4, norm_correction=True,
        mid_o_buf=mid_buf, output_buf=out_buf, lse_buf=lse_buf, buf_holder=Holder(),
        max_num_kv_splits=32)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.data_ptr() == out_buf.data_ptr()
    q_rot = (query.astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    mid = native.stage1(q_rot, cache, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=8,
                        is_aos=layout == "aos")
    ro, rl = native.stage2(mid, w.seq_lens)
    live = w.seq_lens > 0
    err = np.abs(out.float().cpu().numpy()[live] - ro[live]).max()
    print(f"{layout} decode entry fp16 max-abs {err:.3e}")
    assert err <= 1e-3
    assert np.abs(lse_buf[:5].cpu().numpy()[live] - rl[live]).max() <= 1e-4
    with pytest.raises(RuntimeError):  # a 4-bit cache read with 3-bit arguments is rejected
        mod.triton_turboquant_decode_attention(
            t(query), t(cache), t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids),
            128 ** -0.5, mse_bits=3, key_packed_size=50, value_quant_bits=4)
    # with sinks (split 0 starts from the head's sink logit)
    sinks = rng.normal(0.0, 2.0, 32).astype(np.float32)
    out = mod.triton_turboquant_decode_attention(
        t(query), t(cache), t(w.block_table), t(w.seq_lens), t(rot_t.T.copy()), t(w.centroids),
        128 ** -0.5, mse_bits=4, key_packed_size=66, value_quant_bits=4, norm_correction=True,
        max_num_kv_splits=32, sinks=t(sinks))
    torch.cuda.synchronize()
    smid = ostage.stage1(q_rot, cache, w.block_table, w.seq_lens, w.centroids, 32, num_kv_heads=8,
                         is_aos=layout == "aos", sinks=sinks)
    so, _ = ostage.stage2(smid, w.seq_lens)
    err = np.abs(out.float().cpu().numpy() - so).max()
    print(f"{layout} decode entry with sinks fp16 max-abs {err:.3e}")
    assert err <= 1e-3


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_full_decode_fused_one_split_path(dev, out_dtype):
    """B256 x 8 kv-heads: one wave per (sequence, kv-head), so the full step runs one split
    per sequence and the Stage1 kernel writes the output rows itself.  Bit-identical to
    Stage1 with one split + Stage2 (including empty sequences: NaN rows, -inf LSE) and
    within the oracle's fp32 gate plus the output type's rounding."""
    rng = np.random.default_rng(207)
    lens = rng.integers(0, 1500, 256).astype(np.int32)
    lens[[3, 100, 255]] = 0
    lens[[4, 7]] = 1
    w = workloads.small(207, 256, lens, 16)
    query = rng.standard_normal((256, 32, 128)).astype(np.float32)
    rot_t = workloads.random_orthogonal(rng, 128)
    t = lambda a: to_dev(a, dev)  # noqa: E731
    q, r = t(query).half(), t(rot_t)
    cache, bt, sl, cents = t(w.kv_cache), t(w.block_table), t(w.seq_lens), t(w.centroids)
    out, lse = ops.full_decode(q, r, cache, bt, sl, cents, 16, out_dtype=out_dtype)
    q_rot = torch.empty(256, 32, 128, device=dev)
    ops.rotate_query(q, r, q_rot)
    mid = ops.stage1(q_rot, cache, bt, sl, ops.pair_lut_device(cents), num_kv_splits=1)
    ref_out, ref_lse = ops.stage2(mid, sl, out_dtype=out_dtype)
    torch.cuda.synchronize()
    a, b = out.float().cpu().numpy(), ref_out.float().cpu().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.isnan(a[[3, 100, 255]]).all()
    assert np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]), "fused rows differ from Stage1 + Stage2"
    assert np.array_equal(lse.cpu().numpy(), ref_lse.cpu().numpy())
    assert np.isneginf(lse.cpu().numpy()[[3, 100, 255]]).all()
    qr = (query.astype(np.float16).astype(np.float64) @ rot_t.astype(np.float64)).astype(np.float32)
    omid = native.stage1(qr, w.kv_cache, w.block_table, w.seq_lens, w.centroids, 16, num_kv_heads=8)
    ro, _ = native.stage2(omid, w.seq_lens)
    live = lens > 0
    # fp32 gate 1e-4, plus the output type's rounding: unit roundoff 2^-p of its p-bit
    # significand (bf16 p = 8, fp16 p = 11)
    half_ulp = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}[out_dtype]
    excess = np.abs(a[live] - ro[live]) - (1e-4 + half_ulp * np.abs(ro[live]))
    print(f"fused full decode {out_dtype} max-abs {np.abs(a[live] - ro[live]).max():.3e}")
    assert excess.max() <= 0
