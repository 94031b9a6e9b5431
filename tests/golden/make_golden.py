"""Writes the golden fixtures of this directory from the CPU oracle (oracle/), seeded. The reference holds no golden
vectors of its own for this path (its tests gate a real checkpoint by float tolerance), so these vectors are the
oracle's outputs, pinned by tests/test_oracle.py, frozen so that a change to the oracle or to a kernel shows up as
a fixture mismatch. Run from the repository root: python tests/golden/make_golden.py"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import oracle as O  # noqa: E402


def main():
    rng = np.random.default_rng(4242)
    out = {}
    # dequantisation of a 32x48 matrix (2 x 3 tiles) for every compiled (codebook, K2)
    for cb, k2 in sorted(O.COMPILED):
        tr = rng.integers(-32768, 32768, (2, 3, 8 * k2)).astype(np.int16)
        out[f"dequant_cb{cb}_k{k2}_trellis"] = tr
        out[f"dequant_cb{cb}_k{k2}_w"] = O.dequant(tr, k2, cb)
    # input rotation of 3 bf16 rows of 256 with a sign vector
    x = O.f32_to_bf16(rng.standard_normal((3, 256)).astype(np.float32))
    suh = np.where(rng.integers(0, 2, 256) == 1, 1.0, -1.0).astype(np.float16).view(np.uint16)
    out["rotate_x_bf16"], out["rotate_suh"], out["rotate_out"] = x, suh, O.rotate(x, "bf16", suh)
    # had with pre/post scales
    xh = rng.standard_normal((2, 256)).astype(np.float16).view(np.uint16)
    pre = rng.standard_normal(256).astype(np.float16).view(np.uint16)
    post = rng.standard_normal(256).astype(np.float16).view(np.uint16)
    out["had_x"], out["had_pre"], out["had_post"], out["had_out"] = xh, pre, post, O.had(xh, pre, post)
    # exact routing of 4 rows over 64 experts (H 256, top-8) with a tied pair, plus the shared gate
    R, H, E, k = 4, 256, 64, 8
    rx = O.f32_to_bf16(rng.standard_normal((R, H)).astype(np.float32))
    g = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    g[9] = g[5]
    sg = O.f32_to_bf16((rng.standard_normal(H) * 0.02).astype(np.float32))
    pick, wts, logits, sl = O.route(rx, g, k, sg, shared_id=E)
    out.update(route_x=rx, route_gate=g, route_sgate=sg, route_pick=pick, route_wts=wts, route_logits=logits)
    # grouping of a 5 x 9 pick table with repeats and invalid ids
    gp = rng.integers(-1, 12, 45).astype(np.int32)
    cnt, uids, members = O.group(gp, 5, 9, 10, 45)
    out.update(group_pick=gp, group_uids=uids, group_members=members)
    np.savez_compressed(HERE / "oracle_vectors.npz", **out)
    print(f"wrote {len(out)} arrays to {HERE / 'oracle_vectors.npz'}")


if __name__ == "__main__":
    main()
