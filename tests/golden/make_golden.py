"""Write the golden fixtures of tests/golden/ from the reference's own code.

The reference (pure-c-llm) is C: oracle/Makefile compiles its gemm_bench.c,
train.c, transformer.c, model.c and tensor.c where they lie into
oracle/_ref/*.so. This script runs those builds on small seeded inputs and
stores inputs + outputs as .npz (data only, no reference source). The GPU
tests compare libpcl_hip against these files on the GPU box, where the
reference tree does not exist.

Run from the repository root after `make -C oracle`:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import binding as ob  # noqa: E402

p = ob.p


def need(name):
    lib = ob.ref(name)
    if lib is None:
        raise SystemExit(f"oracle/_ref/{name} missing: build it with make -C oracle (needs the reference tree)")
    return lib


def gemm_bench_int8(out):
    gb = need("libref_gemm_bench.so")
    M, K, N = 64, 250, 96  # K not a multiple of 4: exercises Kpad
    Kpad = (K + 3) & ~3
    A = ob.frand((M, K), 101)
    B = ob.frand((K, N), 102)
    Au = np.empty((M, Kpad), np.uint8)
    scale = gb.pcl_ref_quantize_A(p(A), p(Au), M, K, Kpad)
    Bp = np.empty((N // 16) * (Kpad // 4) * 64, np.int8)
    bscale = np.empty(N, np.float32)
    colsum = np.empty(N, np.int32)
    gb.pcl_ref_quantize_B_pack(p(B), p(Bp), p(bscale), p(colsum), K, N, Kpad)
    corr = (128 * colsum).astype(np.int32)
    dq = (np.float32(scale) * bscale).astype(np.float32)
    Cq = np.empty((M, N), np.float32)
    gb.pcl_ref_gemm_int8_kernel(p(Au), Kpad, p(Bp), p(corr), p(dq), p(Cq), M, N)
    Cf = np.empty((M, N), np.float32)
    gb.pcl_ref_gemm_ikj(p(A), p(B), p(Cf), M, K, N)
    np.savez_compressed(out, A=A, B=B, Au=Au, scale=np.float32(scale), Bp=Bp, bscale=bscale,
                        colsum=colsum, corr=corr, dq=dq, C_int8=Cq, C_f32=Cf,
                        dims=np.array([M, K, N, Kpad], np.int32))


def matmul_f32(out):
    md = need("libref_model.so")
    res = {}
    for (M, K, N), seed in (((17, 33, 65), 201), ((64, 64, 64), 211), ((1, 130, 7), 221)):
        A = ob.frand((M, K), seed)
        B = ob.frand((K, N), seed + 1)
        Cm = np.empty((M, N), np.float32)
        md.matmul(p(A), p(B), p(Cm), M, K, N)
        tag = f"{M}x{K}x{N}"
        res[f"A_{tag}"], res[f"B_{tag}"], res[f"C_{tag}"] = A, B, Cm
    np.savez_compressed(out, **res)


def train_gemms(out):
    tr = need("libref_train.so")
    D, V = tr.pcl_ref_train_d_model(), tr.pcl_ref_train_vocab()
    M, K, N = 24, 40, 56
    X = ob.normal((M, K), 301)
    W = ob.normal((K, N), 302, 0.0, 0.02)
    bias = ob.normal((N,), 303, 0.0, 0.1)
    Y = np.empty((M, N), np.float32)
    tr.pcl_ref_matmul_forward(p(Y), p(X), p(W), p(bias), M, K, N)
    dY = ob.normal((M, N), 304, 0.0, 1e-3)
    dX0 = ob.normal((M, K), 305, 0.0, 1e-3)
    dW0 = ob.normal((K, N), 306, 0.0, 1e-3)
    db0 = ob.normal((N,), 307, 0.0, 1e-3)
    dX, dW, db = dX0.copy(), dW0.copy(), db0.copy()
    tr.pcl_ref_matmul_backward(p(dY), p(X), p(W), p(dX), p(dW), p(db), M, K, N)
    Mh = 12
    lnf = ob.normal((Mh, D), 311)
    wte = ob.normal((V, D), 312, 0.0, 0.02)
    logits = np.empty((Mh, V), np.float32)
    tr.pcl_ref_tied_head_forward(p(logits), p(lnf), p(wte), Mh)
    dlog = ob.normal((Mh, V), 313, 0.0, 1e-3)
    dlnf = np.full((Mh, D), 7.0, np.float32)  # SET semantics: must be overwritten
    dwte0 = ob.normal((V, D), 314, 0.0, 1e-3)
    dwte = dwte0.copy()
    tr.pcl_ref_tied_head_backward(p(dlnf), p(dwte), p(dlog), p(lnf), p(wte), Mh)
    np.savez_compressed(out, X=X, W=W, bias=bias, Y=Y, dY=dY, dX0=dX0, dW0=dW0, db0=db0, dX=dX,
                        dW=dW, db=db, lnf=lnf, wte=wte, logits=logits, dlog=dlog, dlnf=dlnf,
                        dwte0=dwte0, dwte=dwte, dims=np.array([M, K, N, Mh, D, V], np.int32))


def decode(out):
    md = need("libref_model.so")
    D, V = md.pcl_ref_model_d_model(), 2048
    K, N = 96, 200
    x = ob.normal((K,), 401)
    W = ob.normal((K, N), 402, 0.0, 0.02)
    b = ob.normal((N,), 403, 0.0, 0.1)
    y = np.empty(N, np.float32)
    md.pcl_ref_proj_token(p(y), p(x), p(W), p(b), K, N)
    T = 2
    # model.c fixes D=1536, V=2048: the 12 MB wte is regenerated from its seed
    # by the oracle PRNG; the fixture keeps seeds, an input digest and outputs.
    xs = ob.normal((T, D), 404)
    wte = ob.normal((V, D), 405, 0.0, 0.02)
    logits = np.empty((T, V), np.float32)
    md.lm_head(p(logits), p(xs), p(wte), T)
    digest = np.frombuffer(hashlib.sha256(xs.tobytes() + wte.tobytes()).digest(), np.uint8)
    np.savez_compressed(out, x=x, W=W, b=b, y=y, logits=logits, head_seeds=np.array([404, 405], np.int32),
                        head_input_sha256=digest, dims=np.array([K, N, T, D, V], np.int32))


if __name__ == "__main__":
    gemm_bench_int8(os.path.join(HERE, "gemm_bench_int8.npz"))
    matmul_f32(os.path.join(HERE, "tensor_matmul_f32.npz"))
    train_gemms(os.path.join(HERE, "train_gemms.npz"))
    decode(os.path.join(HERE, "decode_gemv.npz"))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
