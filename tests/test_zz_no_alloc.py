"""rf_attention_decode_noalloc: the attention entry point that allocates
nothing (split records in the library's static per-device scratch array).

Its output must equal rf_attention_decode's on the same inputs, bit for bit
(same kernels, same launch regime), and meet the oracle bar of the attention
tests; two calls in a row, the second smaller, so the second reads scratch
that still holds the first call's records.  Shapes whose scratch need exceeds
the array are refused, and no call changes the VRAM ledger."""
import numpy as np
import pytest

from helpers import assert_close_scaled

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _inputs(rng, hist, qh, kvh, hd):
    return [rng.normal(0, 1, n).astype(np.float32)
            for n in (qh * hd, max(hist, 1) * kvh * hd, max(hist, 1) * kvh * hd, kvh * hd, kvh * hd)]


def _scale(q, kh, vh, kc, vc, hist, qh, kvh, hd):
    """sum_p softmax_p |v_p| per output element (float64): the attention
    tests' term magnitude."""
    K = np.concatenate([kh[:hist * kvh * hd].reshape(hist, kvh, hd), kc.reshape(1, kvh, hd)]).astype(np.float64)
    V = np.concatenate([vh[:hist * kvh * hd].reshape(hist, kvh, hd), vc.reshape(1, kvh, hd)]).astype(np.float64)
    out = np.zeros((qh, hd))
    for h in range(qh):
        g = h * kvh // qh
        s = K[:, g] @ q.reshape(qh, hd)[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ np.abs(V[:, g])
    return out.reshape(-1)


@pytest.mark.parametrize("shapes", [
    [(8191, 32, 8, 128), (300, 32, 8, 128)],   # per-KV-head split, then per-query-head split
    [(2047, 32, 8, 128), (40, 32, 8, 128)],    # split + merge, then one chunk without merge
    [(700, 6, 3, 10), (9, 6, 3, 10)],          # the any-shape kernel (score rows in scratch)
], ids=["8192-then-301", "2048-then-41", "any-shape"])
def test_noalloc_matches_attention_decode(ctx, orc, shapes):
    import ramforge_amd as rf

    rng = np.random.default_rng(4242)
    used = ctx.vram_used
    for hist, qh, kvh, hd in shapes:
        print(f"  noalloc attention hist={hist} qh={qh} kvh={kvh} hd={hd}", flush=True)
        host = _inputs(rng, hist, qh, kvh, hd)
        dev = [ctx.array(a) for a in host]
        out_ref = rf.attention_checked(ctx, *dev, hist, qh, kvh, hd)
        ref_bits = out_ref.numpy()
        out = ctx.empty((qh * hd,))
        out.upload(np.full(qh * hd, np.nan, np.float32))
        used = ctx.vram_used  # after the workspace path's own growth and the output buffer
        rf.attention_checked_noalloc(ctx, *dev, hist, qh, kvh, hd, out)
        got = out.numpy()
        assert ctx.vram_used == used, "the no-allocation entry point charged device memory"
        assert np.array_equal(got.view(np.uint32), ref_bits.view(np.uint32)), "differs from rf_attention_decode"
        q, kh, vh, kc, vc = host
        ref = orc.attention(q, kh[:hist * kvh * hd], vh[:hist * kvh * hd], kc, vc, hist, qh, kvh, hd)
        assert_close_scaled(got, ref, _scale(q, kh, vh, kc, vc, hist, qh, kvh, hd), TOL,
                            what=f"noalloc attention hist={hist}")
        for a in dev + [out, out_ref]:
            a.free()


def test_noalloc_refuses_oversized_scratch(ctx):
    import ramforge_amd as rf

    # the any-shape kernel keeps qh x (hist + 1) scores: 64 heads x 40000
    # positions = 10 MB, more than the 8 MiB array; nothing is launched
    qh, kvh, hd, hist = 64, 64, 10, 39999
    z = ctx.empty((hist * kvh * hd,))
    small = ctx.empty((qh * hd,))
    out = ctx.empty((qh * hd,))
    with pytest.raises(rf.RamforgeError, match="scratch"):
        rf.attention_checked_noalloc(ctx, small, z, z, small, small, hist, qh, kvh, hd, out)
    for a in (z, small, out):
        a.free()
