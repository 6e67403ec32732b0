"""The reference's own CPU kernels, built from knn.cpp and fps.cpp where they
lie in the reference checkout (oracle/ref.mk -> oracle/_ref/), against

  - the oracle's restatement of them (tpo_cpu_*, oracle/tpo_oracle.c), which
    bench.py times as the CPU baseline, and
  - the product's CPU dispatch keys (csrc/cpu_ops.cpp),

bit for bit: KNN forward and backward (knn.cpp:30-164, float32/float64/
float16, both norms, ragged lengths, K above the cloud length, lattice
ties), FPS and quick FPS (fps.cpp:18-88, 143-155; degenerate points, ties),
gather_points forward and backward (fps.cpp:91-141).

The reference registers the same torch.library namespaces as the product, so
its kernels run in a child process (tests/ref_cpu_child.py).  Without a
reference checkout and without built kernels the test is skipped."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
REF_DIR = os.path.join(REPO, "oracle", "_ref")
REF_SRC = "/root/reference"

pytestmark = pytest.mark.usefixtures("tpo")  # the product's CPU keys


def _built():
    return all(os.path.exists(os.path.join(REF_DIR, f)) for f in ("knn_ref.so", "fps_ref.so"))


@pytest.fixture(scope="module")
def ref_results(tmp_path_factory):
    if os.path.isdir(REF_SRC):
        subprocess.run(["make", "-s", "-f", os.path.join(REPO, "oracle", "ref.mk"),
                        f"REF={REF_SRC}"], check=True)
    if not _built():
        pytest.skip("no reference checkout and no oracle/_ref build")
    cases, meta = _cases()
    d = tmp_path_factory.mktemp("ref")
    src, dst = str(d / "in.npz"), str(d / "out.npz")
    np.savez(src, **cases)
    env = dict(os.environ, OMP_NUM_THREADS="4")
    subprocess.run([sys.executable, os.path.join(HERE, "ref_cpu_child.py"), REF_DIR, src, dst],
                   check=True, env=env, cwd=str(d))
    return cases, dict(np.load(dst, allow_pickle=False)), meta


def _cases():
    cases, meta = {}, []
    r = np.random.default_rng(77)
    n = 0
    for dt in (np.float32, np.float64, np.float16):
        for norm in (1, 2):
            for K, D, lattice in ((1, 3, False), (5, 3, True), (16, 3, False), (40, 7, False),
                                  (8, 64, False)):
                N, P1, P2 = 3, 60, 90
                if lattice:
                    p1 = r.integers(-3, 4, (N, P1, D)).astype(dt)
                    p2 = r.integers(-3, 4, (N, P2, D)).astype(dt)
                else:
                    p1 = r.standard_normal((N, P1, D)).astype(dt)
                    p2 = r.standard_normal((N, P2, D)).astype(dt)
                l1 = np.array([P1, 41, 1], np.int64)
                l2 = np.array([P2, 3, 70], np.int64)  # 3 < K: padding rows
                key = f"c{n:03d}"
                n += 1
                cases.update({f"{key}.op": np.array("knn"), f"{key}.p1": p1, f"{key}.p2": p2,
                              f"{key}.l1": l1, f"{key}.l2": l2, f"{key}.norm": np.array(norm),
                              f"{key}.K": np.array(K),
                              f"{key}.g": r.standard_normal((N, P1, K)).astype(dt)})
                meta.append((key, "knn", dt, norm, K, D))
    for dt in (np.float32, np.float64, np.float16):
        for kind in ("random", "lattice", "degenerate"):
            if kind == "random":
                pts = r.standard_normal((2, 200, 3))
            elif kind == "lattice":
                pts = r.integers(-2, 3, (2, 125, 3)).astype(np.float64)
            else:
                pts = r.standard_normal((2, 100, 3))
                pts[:, 10:20] = 1e-3 * r.standard_normal((2, 10, 3))
                pts[:, 0] = 0.0
            key = f"c{n:03d}"
            n += 1
            m = 40
            cases.update({f"{key}.op": np.array("fps"), f"{key}.pts": pts.astype(dt),
                          f"{key}.m": np.array(m)})
            meta.append((key, "fps", dt, kind, m))
        key = f"c{n:03d}"
        n += 1
        B, C, Np, M = 2, 5, 70, 30
        idx = r.integers(0, Np, (B, M)).astype(np.int64)
        idx[:, :4] = 7  # repeated indices accumulate in the backward
        cases.update({f"{key}.op": np.array("gather"),
                      f"{key}.feat": r.standard_normal((B, C, Np)).astype(dt),
                      f"{key}.idx": idx, f"{key}.gout": r.standard_normal((B, C, M)).astype(dt),
                      f"{key}.n": np.array(Np)})
        meta.append((key, "gather", dt))
    return cases, meta


def bits(a):
    a = a.detach().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    return a.view(np.uint8)


def same(a, b):
    return np.asarray(a).shape == np.asarray(b).shape and np.array_equal(bits(a), bits(b))


def test_knn_reference_cpu_kernel(O, ref_results):
    cases, out, meta = ref_results
    for key, op, *rest in meta:
        if op != "knn":
            continue
        c = {k.split(".", 1)[1]: v for k, v in cases.items() if k.startswith(key + ".")}
        norm, K = int(c["norm"]), int(c["K"])
        ri, rd, rg1, rg2 = (out[f"{key}.{x}"] for x in ("idx", "d", "g1", "g2"))
        # the oracle's restatement (the timed CPU baseline)
        ei, ed = O.cpu_knn_fwd(c["p1"], c["p2"], c["l1"], c["l2"], K, norm)
        assert same(ei, ri) and same(ed, rd), (key, rest)
        e1, e2 = O.cpu_knn_bwd(c["p1"], c["p2"], c["l1"], c["l2"], ri, norm, c["g"])
        assert same(e1, rg1) and same(e2, rg2), (key, rest)
        # the product's CPU keys
        t = {k: torch.from_numpy(v) for k, v in c.items() if k in ("p1", "p2", "l1", "l2", "g")}
        pi, pd = torch.ops.torch_point_ops_knn.knn_forward(t["p1"], t["p2"], t["l1"], t["l2"],
                                                            norm, K, -1)
        assert same(pi, ri) and same(pd, rd), (key, rest)
        p1g, p2g = torch.ops.torch_point_ops_knn.knn_backward(t["p1"], t["p2"], t["l1"], t["l2"],
                                                               pi, norm, t["g"])
        assert same(p1g, rg1) and same(p2g, rg2), (key, rest)


def test_fps_and_gather_reference_cpu_kernels(O, ref_results):
    cases, out, meta = ref_results
    for key, op, dt, *rest in meta:
        if op == "fps":
            pts, m = cases[f"{key}.pts"], int(cases[f"{key}.m"])
            ref = out[f"{key}.idx"]
            assert same(out[f"{key}.qidx"], ref), key
            assert same(O.cpu_fps(pts, m), ref), (key, dt, rest)
            t = torch.from_numpy(pts)
            assert same(torch.ops.torch_point_ops_fps.fps_forward(t, m), ref), (key, dt, rest)
            assert same(torch.ops.torch_point_ops_quick_fps.quick_fps_forward(t, m, 4), ref)
        elif op == "gather":
            feat, idx, gout = (cases[f"{key}.{x}"] for x in ("feat", "idx", "gout"))
            n = int(cases[f"{key}.n"])
            assert same(O.cpu_gather_fwd(feat, idx), out[f"{key}.fwd"]), (key, dt)
            assert same(O.cpu_gather_bwd(gout, idx, n), out[f"{key}.bwd"]), (key, dt)
            tf, ti, tg = (torch.from_numpy(x) for x in (feat, idx, gout))
            assert same(torch.ops.torch_point_ops_fps.gather_points_forward(tf, ti),
                        out[f"{key}.fwd"]), (key, dt)
            assert same(torch.ops.torch_point_ops_fps.gather_points_backward(tg, ti, n),
                        out[f"{key}.bwd"]), (key, dt)
