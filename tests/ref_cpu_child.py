"""Child process of tests/test_ref_cpu_kernels.py: loads the reference's own
CPU kernels (oracle/_ref/*.so, built from knn.cpp and fps.cpp by
oracle/ref.mk) and runs them on the inputs the parent wrote.

They register the torch.library namespaces the product registers
(torch_point_ops_knn, _fps, _quick_fps), so they run in a process of their
own, which imports nothing else of this repository.

    python ref_cpu_child.py <ref dir> <inputs.npz> <outputs.npz>
"""
import sys

import numpy as np
import torch


def main(ref_dir, src, dst):
    torch.ops.load_library(f"{ref_dir}/knn_ref.so")
    torch.ops.load_library(f"{ref_dir}/fps_ref.so")
    cases = dict(np.load(src, allow_pickle=False))
    out = {}
    for key in sorted(k[:-3] for k in cases if k.endswith(".op")):
        op = str(cases[key + ".op"])
        t = lambda name: torch.from_numpy(cases[f"{key}.{name}"])
        i = lambda name: int(cases[f"{key}.{name}"])
        if op == "knn":
            idx, d = torch.ops.torch_point_ops_knn.knn_forward(
                t("p1"), t("p2"), t("l1"), t("l2"), i("norm"), i("K"), -1)
            g1, g2 = torch.ops.torch_point_ops_knn.knn_backward(
                t("p1"), t("p2"), t("l1"), t("l2"), idx, i("norm"), t("g"))
            out.update({f"{key}.idx": idx.numpy(), f"{key}.d": d.numpy(),
                        f"{key}.g1": g1.numpy(), f"{key}.g2": g2.numpy()})
        elif op == "fps":
            out[f"{key}.idx"] = torch.ops.torch_point_ops_fps.fps_forward(t("pts"), i("m")).numpy()
            out[f"{key}.qidx"] = torch.ops.torch_point_ops_quick_fps.quick_fps_forward(
                t("pts"), i("m"), 4).numpy()
        elif op == "gather":
            out[f"{key}.fwd"] = torch.ops.torch_point_ops_fps.gather_points_forward(
                t("feat"), t("idx")).numpy()
            out[f"{key}.bwd"] = torch.ops.torch_point_ops_fps.gather_points_backward(
                t("gout"), t("idx"), i("n")).numpy()
        else:
            raise ValueError(op)
    np.savez(dst, **out)


if __name__ == "__main__":
    main(*sys.argv[1:4])
