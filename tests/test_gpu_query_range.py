"""bf16 queries beyond the fp16 range.

Both attention kernels take the queries as fp16.  A bf16 query row whose
largest |q| is at or above 65504 would round to inf there (and its scores to
NaN); such a row is scaled by an exact power of two 2^-k before the rounding
and its scores by 2^k.  The reference computes these scores in bf16/fp32 SDPA
(MLXFast.scaledDotProductAttention, Attention.swift:95-98,
Gemma4Model.swift:516-517), where nothing overflows.

Exactness makes the check bit for bit, with no tolerance: multiplying a row
by 2^17 and its scale by 2^-17 leaves every score, and so the output,
unchanged.  One call mixes such rows (odd query heads) with ordinary rows
(even heads):
- its even heads must equal those of the call on the unscaled queries;
- its odd heads must equal those of the call on the unscaled queries with
  the scale x 2^17 (the same mathematical scores, reached without a large
  query).
The unscaled call is checked against the float64 oracle at 2e-3 max-abs.
Query elements below 1e-3 in magnitude are moved to +-1e-3 so that no element
is an fp16 subnormal in one call and a normal number in the other."""
import numpy as np
import pytest

from kvutil import Filled, oracle_attention, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from oracle import oracle as O  # noqa: E402

ATOL = 2e-3
BIG = 2.0 ** 17


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,Lq,path", [(128, 1, 1), (512, 1, 1), (128, 8, 0), (256, 8, 0)],
                         ids=["decode-d128", "decode-d512", "verify-d128", "verify-d256"])
def test_query_rows_beyond_fp16_range(mode, D, Lq, path):
    print(f"\ncase query-range mode={mode} D={D} Lq={Lq} path={path}", flush=True)
    H, R = 2, (4 if Lq == 1 else 2)
    lens = [300, 900]
    rng = np.random.default_rng(2100 + D + Lq)
    pool = krill_amd.KVPool(1, H, D, sum((T + 63) // 64 for T in lens) + 8, mode, "bf16", free_list_seed=7)
    pool.set_option(krill_amd._lib.OPT_ATTN_PATH, path)
    f = Filled(pool, lens, rng, "bf16")
    tables, tl, _ = f.tables()
    B = len(lens)
    q = rng.standard_normal((B, H * R, Lq, D)).astype(np.float32)
    q = np.where(np.abs(q) < 1e-3, np.copysign(1e-3, q), q)
    q0 = O.f32_to_bf16_bits(q)
    qf = O.bits_to_f32(q0, O.DT_BF16)
    mixed = qf.copy()
    mixed[:, 1::2] *= BIG  # exact in bf16: a power of two
    qm = O.f32_to_bf16_bits(mixed)
    assert np.array_equal(O.bits_to_f32(qm, O.DT_BF16)[:, 1::2], qf[:, 1::2] * BIG)
    assert np.abs(O.bits_to_f32(qm, O.DT_BF16)).max() > 65504.0

    scale = np.float32(1.0 / np.sqrt(D))
    mx = max(lens)

    def run(qbits, sc):
        out = pool.attention(0, to_dev(qbits, "bf16"), tables, tl, mx, float(sc))
        torch.cuda.synchronize()
        return out.float().cpu().numpy()

    plain = run(q0, scale)
    wide = run(qm, scale)
    plain_big = run(q0, np.float32(scale * np.float32(BIG)))
    ref = oracle_attention(pool, f, 0, q0, "bf16", float(scale))
    pool.close()

    assert np.isfinite(wide).all(), "non-finite output for rows beyond the fp16 range"
    err = np.abs(plain - ref).max()
    print(f"unscaled call against the oracle: max abs error {err:.3e}", flush=True)
    assert err <= ATOL
    assert np.array_equal(wide[:, 0::2], plain[:, 0::2]), "ordinary rows changed"
    assert np.array_equal(wide[:, 1::2], plain_big[:, 1::2]), "scaled rows differ from the same scores at scale x 2^17"
