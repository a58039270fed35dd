"""Write the golden fixtures under tests/golden/ (run in the survey container).

Three kinds of data, none of it reference source:

1. ``dlinoss_reference_cases.json`` — the reference's own layer-level D-LinOSS
   fixture (tests/dlinoss_reference_cases.json: 4 variants x fp32/fp64, B=1,
   L=6, P=4, H=3, states and gradients), copied as data.
2. ``linoss_reference_snapshot.json`` — the numbers of the reference's
   ``REFERENCE_LINOSS`` LinOSS-IM layer snapshot (tests/test_linoss_parity.py:74-204),
   read as text with ``ast`` and stored as plain lists.
3. ``ref_kernel_vectors.npz`` — inputs and outputs of the reference's own CPU
   kernels (``oracle/_ref``, compiled from src/ossm/csrc by oracle/Makefile.ref)
   on small seeded cases: D-LinOSS forward/backward for every variant, LinOSS
   scan forward, selective scan forward/backward with and without the gate.
4. ``sdl_kernel_vectors.npz`` — the same for the selective D-LinOSS kernels
   (every variant, every accepted parameter layout, both clamps exercised).
5. ``diag_kernel_vectors.npz`` — the reference's ``lru_scan`` and ``s5_scan`` CPU
   kernels (lru_scan.cpp, s5_scan.cpp) in fp32 and fp64 on a ragged shape.
6. ``complex_scan_reference.json`` — the numbers of the reference's
   ``REFERENCE_COMPLEX_{LAMBDA,B,STATES}`` (tests/test_scan_parity.py:186-349),
   read as text with ``ast`` and stored as [re, im] pairs.

Usage (from the repository root, with /root/reference present and
``make -f oracle/Makefile.ref`` done):

    python tests/golden/make_golden.py [dlinoss] [linoss] [kernels] [sdlinoss] [diag] [complex]

(no argument: all).  The reference's OpenMP kernels add some sums in a
thread-dependent order, so regenerating a fixture changes its last bits.
"""

from __future__ import annotations

import ast
import json
import shutil
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent


def _copy_dlinoss_fixture() -> None:
    src = REF / "tests" / "dlinoss_reference_cases.json"
    shutil.copyfile(src, OUT / "dlinoss_reference_cases.json")


def _tensor_literal(node: ast.AST):
    """Return the literal data of a ``torch.tensor([...])`` call node."""
    if isinstance(node, ast.Call) and node.args:
        return ast.literal_eval(node.args[0])
    return ast.literal_eval(node)


def _extract_linoss_snapshot() -> None:
    text = (REF / "tests" / "test_linoss_parity.py").read_text()
    tree = ast.parse(text)
    snapshot = None
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(
            isinstance(t, ast.Name) and t.id == "REFERENCE_LINOSS" for t in node.targets
        ):
            snapshot = node.value
    assert isinstance(snapshot, ast.Dict), "REFERENCE_LINOSS literal not found"
    data = {}
    for key, value in zip(snapshot.keys, snapshot.values):
        data[ast.literal_eval(key)] = _tensor_literal(value)
    data["_provenance"] = (
        "numbers of REFERENCE_LINOSS, reference tests/test_linoss_parity.py:74-204; "
        "LinOSSLayer(4, 6, 'IM'); C is stored flat and viewed as (6, 4, 2) by the test (:196)"
    )
    (OUT / "linoss_reference_snapshot.json").write_text(json.dumps(data))


def _ref_kernel_vectors() -> None:
    import torch

    import oracle

    ref = oracle.reference_module()
    assert ref is not None, "build oracle/_ref first: make -f oracle/Makefile.ref"
    rng = np.random.default_rng(20240601)
    vec: dict[str, np.ndarray] = {}
    T = torch.from_numpy

    # D-LinOSS: ragged shape (P not a multiple of anything, L odd), fp32.
    L, B, P = 53, 3, 7
    a = rng.uniform(0.1, 1.0, P).astype(np.float32)
    g = rng.uniform(0.0, 1.0, P).astype(np.float32)
    dt = (1.0 / (1.0 + np.exp(-rng.normal(size=P)))).astype(np.float32)
    bu = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    go = (rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))).astype(np.complex64)
    vec.update(dl_a=a, dl_g=g, dl_step=dt, dl_bu=bu, dl_grad=go)
    for v in oracle.VARIANTS:
        st = getattr(ref, f"dlinoss_{v}_forward")(T(a), T(g), T(dt), T(bu)).numpy()
        ga, gg, gs, gb = (x.numpy() for x in getattr(ref, f"dlinoss_{v}_backward")(
            T(a), T(g), T(dt), T(bu), T(st), T(go)))
        vec[f"dl_{v}_states"] = st
        vec[f"dl_{v}_grad_a"], vec[f"dl_{v}_grad_g"] = ga, gg
        vec[f"dl_{v}_grad_step"], vec[f"dl_{v}_grad_bu"] = gs, gb

    # LinOSS: complex M with spectral radius < 1 so states stay O(1).
    L, B, P = 41, 2, 5
    ms = []
    for _ in range(4):
        ms.append(((rng.normal(size=P) + 1j * rng.normal(size=P)) * 0.35).astype(np.complex64))
    bs = (rng.normal(size=(L, B, P, 2)) + 1j * rng.normal(size=(L, B, P, 2))).astype(np.complex64)
    out = ref.linoss_scan(*[T(m) for m in ms], T(bs)).numpy()
    vec.update(lo_m11=ms[0], lo_m12=ms[1], lo_m21=ms[2], lo_m22=ms[3], lo_b=bs, lo_out=out)

    # Selective scan: distributions of the reference tests (test_scan_parity.py:63-135).
    Bz, D, Ls, N = 2, 5, 47, 8
    u = rng.normal(size=(Bz, D, Ls)).astype(np.float32)
    dts = (rng.uniform(size=(Bz, D, Ls)) * 0.05).astype(np.float32)
    A = (-np.exp(rng.normal(size=(D, N)))).astype(np.float32)
    Bm = rng.normal(size=(Bz, Ls, N)).astype(np.float32)
    Cm = rng.normal(size=(Bz, Ls, N)).astype(np.float32)
    z = rng.normal(size=(Bz, D, Ls)).astype(np.float32)
    gs = rng.normal(size=(Bz, D, Ls)).astype(np.float32)
    vec.update(sel_u=u, sel_dt=dts, sel_A=A, sel_B=Bm, sel_C=Cm, sel_z=z, sel_grad=gs)
    for tag, gate in (("gate", z), ("nogate", None)):
        gt = None if gate is None else T(gate)
        y = ref.selective_scan(T(u), T(dts), T(A), T(Bm), T(Cm), gt).numpy()
        grads = [x.numpy() for x in ref.selective_scan_backward(
            T(gs), T(u), T(dts), T(A), T(Bm), T(Cm), gt)]
        vec[f"sel_{tag}_out"] = y
        for name, arr in zip(("du", "ddt", "dA", "dB", "dC", "dz"), grads):
            vec[f"sel_{tag}_{name}"] = arr

    np.savez_compressed(OUT / "ref_kernel_vectors.npz", **vec)


def _sdl_kernel_vectors() -> None:
    """Selective D-LinOSS: the reference's CPU kernels (sdlinoss_<v>.cpp) on a
    ragged shape with every parameter layout the kernels accept, with steps and
    stiffnesses that hit both clamps (dt outside (1e-6, 1), S below 1e-6)."""
    import torch

    import oracle

    ref = oracle.reference_module()
    assert ref is not None, "build oracle/_ref first: make -f oracle/Makefile.ref"
    rng = np.random.default_rng(20241130)
    T = torch.from_numpy
    L, B, M = 29, 2, 5
    vec: dict[str, np.ndarray] = {}
    bu = (rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))).astype(np.complex64)
    go = (rng.normal(size=(L, B, M)) + 1j * rng.normal(size=(L, B, M))).astype(np.complex64)
    vec.update(bu=bu, grad=go)
    shapes = {"full": (L, B, M), "bcast_t": (1, B, M), "bcast_b": (L, 1, M), "m": (M,)}
    for v in oracle.VARIANTS:
        for tag, shp in shapes.items():
            if tag != "full" and v in ("imex2", "ex"):
                continue
            A = rng.uniform(0.1, 1.5, shp).astype(np.float32)
            G = rng.uniform(0.0, 1.0, shp).astype(np.float32)
            S = rng.uniform(-0.2, 1.3, shp).astype(np.float32)  # clamps dt on both sides
            if v in ("imex1", "im") and len(shp) == 3 and shp[0] == L:
                # S = 1 + dt g (+ dt^2 a) below the 1e-6 clamp, at the last step only
                # (earlier, the 1e6 gain would overflow the rest of the sequence)
                G[-1, :, ::2] = -3.0
                S[-1, :, ::2] = 0.9
            st = getattr(ref, f"sdlinoss_{v}_forward")(T(A), T(G), T(S), T(bu)).numpy()
            ga, gg, gs, gb = (x.numpy() for x in getattr(ref, f"sdlinoss_{v}_backward")(
                T(A), T(G), T(S), T(bu), T(st), T(go)))
            key = f"{v}_{tag}"
            vec.update({f"{key}_A": A, f"{key}_G": G, f"{key}_step": S, f"{key}_states": st,
                        f"{key}_grad_A": ga, f"{key}_grad_G": gg, f"{key}_grad_step": gs,
                        f"{key}_grad_bu": gb})
    np.savez_compressed(OUT / "sdl_kernel_vectors.npz", **vec)


def _diag_kernel_vectors() -> None:
    """Diagonal scans: lru_scan / s5_scan of the reference's CPU build on a ragged
    shape, eigenvalues inside the unit disc (some close to it, some negative or
    purely imaginary), in fp32 and fp64."""
    import torch

    import oracle

    ref = oracle.reference_module()
    assert ref is not None, "build oracle/_ref first: make -f oracle/Makefile.ref"
    rng = np.random.default_rng(20240611)
    L, B, P = 37, 3, 7
    radius = np.array([0.0, 0.3, 0.9, 0.99, 0.999, 0.6, 0.5])
    angle = np.array([0.0, 2.5, -0.4, 0.05, np.pi, np.pi / 2, -3.0])
    lam = radius * np.exp(1j * angle)
    b = rng.normal(size=(L, B, P)) + 1j * rng.normal(size=(L, B, P))
    vec: dict[str, np.ndarray] = {}
    for prec, ct in (("f32", np.complex64), ("f64", np.complex128)):
        lc = lam.astype(ct)
        bc = b.astype(ct)
        T = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
        args = (T(lc.real), T(lc.imag), torch.view_as_real(T(bc)).contiguous())
        vec[f"{prec}_lambda"], vec[f"{prec}_b"] = lc, bc
        vec[f"{prec}_lru"] = torch.view_as_complex(ref.lru_scan(*args).contiguous()).numpy()
        vec[f"{prec}_s5"] = torch.view_as_complex(ref.s5_scan(*args).contiguous()).numpy()
    np.savez_compressed(OUT / "diag_kernel_vectors.npz", **vec)


def _extract_complex_reference() -> None:
    text = (REF / "tests" / "test_scan_parity.py").read_text()
    tree = ast.parse(text)
    want = ("REFERENCE_COMPLEX_LAMBDA", "REFERENCE_COMPLEX_B", "REFERENCE_COMPLEX_STATES")
    data = {}
    for node in tree.body:
        if isinstance(node, ast.Assign):
            for t in node.targets:
                if isinstance(t, ast.Name) and t.id in want:
                    arr = np.asarray(_tensor_literal(node.value), dtype=np.complex128)
                    data[t.id] = np.stack([arr.real, arr.imag], axis=-1).tolist()
    assert set(data) == set(want), f"literals not found: {set(want) - set(data)}"
    data["_provenance"] = (
        "numbers of REFERENCE_COMPLEX_LAMBDA / _B / _STATES, reference "
        "tests/test_scan_parity.py:186-349 (complex64 literals, stored as [re, im]); "
        "states = lru_scan / s5_scan of lambda over b (test at :465-474, atol=rtol=5e-6)"
    )
    (OUT / "complex_scan_reference.json").write_text(json.dumps(data))


def main() -> None:
    only = sys.argv[1:]
    if not only or "dlinoss" in only:
        _copy_dlinoss_fixture()
    if not only or "linoss" in only:
        _extract_linoss_snapshot()
    if not only or "kernels" in only:
        _ref_kernel_vectors()
    if not only or "sdlinoss" in only:
        _sdl_kernel_vectors()
    if not only or "diag" in only:
        _diag_kernel_vectors()
    if not only or "complex" in only:
        _extract_complex_reference()
    for p in sorted(OUT.iterdir()):
        print(f"{p.name:40s} {p.stat().st_size:>10d} B")


if __name__ == "__main__":
    main()
