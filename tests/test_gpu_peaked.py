"""GPU parity of attention when a few keys dominate the softmax.

Queries built from chosen keys' dequantized rows put almost all of the
softmax weight on one to three keys, so the output is close to those keys'
value rows and every rounding of the value weights shows at full size (a
diffuse softmax averages such errors away).  Variants: one key, three keys
of comparable weight, the same with x20 outlier channels in K and V (the
long-context MoE shape's stress case), and random queries scaled x30 (very
large scores).  Each case runs on the VALU decode path and the MFMA verify
path, in both storage modes, against the float64 oracle at 2e-3 max-abs
(float32 output).  The reference computes these outputs with fp32-weight
SDPA (MLXFast.scaledDotProductAttention, Attention.swift:95-98,
Gemma4Model.swift:516-517)."""
import numpy as np
import pytest

from kvutil import DT, MODE, Filled, oracle_attention, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from oracle import oracle as O  # noqa: E402

ATOL = 2e-3


def _peaked_queries(f, pool, dt, Lq, R, variant, rng):
    """q [B, Hq, Lq, D] (dtype bits) whose rows point at chosen keys."""
    B, H, D = len(f.lens), pool.num_kv_heads, pool.head_dim
    mode = MODE[pool.quant_mode]
    q = np.zeros((B, H * R, Lq, D), np.float32)
    # scores (after the 1/sqrt(D) scale) the hot keys get, in nats: far above
    # every other key's, and within 1.4 of each other, so the three share the
    # weight about 57 / 29 / 14 %
    targets = np.array([24.0, 23.3, 22.6]) * np.sqrt(D)
    for b, T in enumerate(f.lens):
        kq, ks, kz, _, _, _ = f.expected(0, b)
        kd = O.dequant_f64(kq, ks, kz, mode)  # [H, T, D]
        for hk in range(H):
            # channels of ordinary size: the query stays off the x20 outlier
            # channels, so that the other keys' scores stay ordinary too
            keep = (kd[hk].std(axis=0) < 5.0).astype(np.float64)
            for r in range(R * Lq):
                hq, j = hk * R + r % R, r // R
                visible = T - Lq + j + 1
                if variant == "q_x30":
                    q[b, hq, j] = rng.standard_normal(D) * 30.0
                    continue
                n_hot = 1 if variant == "one_key" else 3
                hot = rng.choice(visible, size=n_hot, replace=False)
                Kh = kd[hk, hot] * keep
                # the query in the span of the hot keys with exactly the target scores
                a = np.linalg.solve(Kh @ Kh.T, targets[:n_hot])
                q[b, hq, j] = a @ Kh
    return O.f32_to_bf16_bits(q) if dt == "bf16" else O.f32_to_f16_bits(q)


def _top_mass(pool, f, q_bits, dt, scale, Lq, R, k=3):
    """Smallest, over all query rows, of the softmax mass on the top k keys."""
    mode = MODE[pool.quant_mode]
    qf = O.bits_to_f32(q_bits, DT[dt]).astype(np.float64)
    worst = 1.0
    for b, T in enumerate(f.lens):
        kq, ks, kz, _, _, _ = f.expected(0, b)
        kd = O.dequant_f64(kq, ks, kz, mode)
        for hk in range(pool.num_kv_heads):
            for r in range(R * Lq):
                j = r // R
                s = kd[hk, : T - Lq + j + 1] @ qf[b, hk * R + r % R, j] * scale
                p = np.exp(s - s.max())
                p /= p.sum()
                worst = min(worst, float(np.sort(p)[-k:].sum()))
    return worst


def _case(mode, variant, Lq, path, seed, dt="bf16"):
    H, R, D = 2, (5 if Lq == 1 else 4), 128
    lens = [700, 2100] if Lq == 1 else [1100, 2500]
    rng = np.random.default_rng(seed)
    pool = krill_amd.KVPool(1, H, D, sum((T + 63) // 64 for T in lens) + 8, mode, dt, free_list_seed=seed)
    pool.set_option(krill_amd._lib.OPT_ATTN_PATH, path)
    outl = 0.01 if variant == "three_keys_outliers" else 0.0
    f = Filled(pool, lens, rng, dt, outlier_frac=outl)
    tables, tl, _ = f.tables()
    q = _peaked_queries(f, pool, dt, Lq, R, variant, rng)
    scale = 1.0 / np.sqrt(D)
    out = pool.attention(0, to_dev(q, dt), tables, tl, max(lens), scale)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    mass = _top_mass(pool, f, q, dt, scale, Lq, R)
    pool.close()
    return got, ref, mass


VARIANTS = ["one_key", "three_keys", "three_keys_outliers", "q_x30"]
# random queries x30 concentrate the weight on the largest scores without a
# chosen key: a few keys still hold almost all of it
MIN_MASS = {"one_key": 0.99, "three_keys": 0.99, "three_keys_outliers": 0.99, "q_x30": 0.5}


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_decode_valu_peaked(mode, variant):
    print(f"\ncase peaked decode_valu mode={mode} variant={variant}", flush=True)
    got, ref, mass = _case(mode, variant, 1, 1, seed=300 + VARIANTS.index(variant))
    assert mass > MIN_MASS[variant], f"softmax not peaked: top-3 mass {mass:.4f}"
    err = np.abs(got - ref).max()
    print(f"max abs error {err:.3e} (top-3 mass >= {mass:.4f})", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_verify_mfma_peaked(mode, variant):
    print(f"\ncase peaked verify_mfma mode={mode} variant={variant}", flush=True)
    got, ref, mass = _case(mode, variant, 8, 0, seed=400 + VARIANTS.index(variant))
    assert mass > MIN_MASS[variant], f"softmax not peaked: top-3 mass {mass:.4f}"
    err = np.abs(got - ref).max()
    print(f"max abs error {err:.3e} (top-3 mass >= {mass:.4f})", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("variant", ["three_keys", "three_keys_outliers"])
def test_decode_mfma_forced_peaked(variant):
    print(f"\ncase peaked decode_mfma variant={variant}", flush=True)
    got, ref, mass = _case("affine_g64", variant, 1, 2, seed=500 + VARIANTS.index(variant))
    assert mass > 0.99
    err = np.abs(got - ref).max()
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("mode", ["affine_g64"])
def test_fused_append_of_a_dominant_token(mode):
    """The fused decode step appends a newest token with x20 outlier channels
    that holds most of the softmax weight: the token patched into the
    registers of its block must enter P.V at full weight precision."""
    print("\ncase peaked fused-wide-token", flush=True)
    from kvutil import i32, rand_bits

    dt, H, R, D = "bf16", 2, 5, 128
    lens = [700, 1500]
    rng = np.random.default_rng(808)
    pool = krill_amd.KVPool(1, H, D, sum((T + 64) // 64 for T in lens) + 8, mode, dt, free_list_seed=5)
    pool.set_option(krill_amd._lib.OPT_ATTN_PATH, 1)
    f = Filled(pool, lens, rng, dt)
    B = len(lens)
    kn = rand_bits(rng, (B, H, 1, D), dt, outlier_frac=0.05)
    vn = rand_bits(rng, (B, H, 1, D), dt, outlier_frac=0.05)
    for b in range(B):
        pool.reserve_append(f.seqs[b], 1)
    full = [T + 1 for T in lens]
    # the oracle's view: history plus the new token
    for b in range(B):
        f.k[0][b] = np.concatenate([f.k[0][b], kn[b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], vn[b]], axis=1)
    f.lens = full
    mode_i = MODE[mode]
    targets = np.array([24.0, 23.3, 22.6]) * np.sqrt(D)
    q = np.zeros((B, H * R, 1, D), np.float32)
    for b, T in enumerate(full):
        kq, ks, kz, _, _, _ = f.expected(0, b)
        kd = O.dequant_f64(kq, ks, kz, mode_i)
        for hk in range(H):
            keep = (np.abs(kd[hk, :-1]).std(axis=0) < 5.0).astype(np.float64)
            for r in range(R):
                hot = [T - 1] + list(rng.choice(T - 1, size=2, replace=False))  # the new token first
                Kh = kd[hk, hot] * keep
                q[b, hk * R + r, 0] = np.linalg.solve(Kh @ Kh.T, targets) @ Kh
    qb = O.f32_to_bf16_bits(q)
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in full))
    out = pool.decode_append_attention(0, to_dev(qb, dt), to_dev(kn, dt), to_dev(vn, dt), i32(t), i32(n),
                                       max(full), 1.0 / np.sqrt(D))
    torch.cuda.synchronize()
    ref = oracle_attention(pool, f, 0, qb, dt, 1.0 / np.sqrt(D))
    err = np.abs(out.float().cpu().numpy() - ref).max()
    print(f"max abs error {err:.3e}", flush=True)
    pool.close()
    assert err <= ATOL, f"max abs error {err:.3e}"
