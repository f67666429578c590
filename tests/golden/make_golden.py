"""Write the golden fixtures in this directory from the reference's own ops.

Runs where /root/reference exists: it calls the reference train_bnn.c ops,
compiled unmodified from /root/reference by `make -C oracle ref` into
oracle/_ref/libtrain_bnn.so, on seeded inputs, and stores inputs and outputs
as .npz (plus a sha256 of every output array in golden.json). The GPU box
never runs this script; the tests read the committed files.

    make -C oracle ref && python tests/golden/make_golden.py

Fixtures (shapes are the reference's CPU-runnable configuration, C=384, V=27,
B=4, T=64, and the 256x384 LayerNorm of benchmark config 2):
  encoder.npz     encoder fwd + bwd, B=4 T=64 C=384 V=27, uniform tokens, plus
                  the repeated-token case of train_bnn.c:1236-1238 (tokens
                  5,2,5,0,5,6 at B=2 T=3 C=4 V=7)
  layernorm.npz   LN fwd + bwd, 256 x 384, accumulators start nonzero
  gelu.npz        GELU fwd + bwd, 65,536 N(0,1) values + special values
  residual.npz    residual fwd + bwd, 65,536 values
  materialize.npz bayes_materialize, 65,536 values + special rho/eps cases
  head.npz        softmax_crossentropy + crossentropy_softmax_backward at
                  B=4 T=64 V=27 (config 1) and B=1 T=2 V=50257
  posterior.npz   bayes_backward, kl_forward, kl_backward and adamw_update
                  (t = 1 and t = 7, with weight decay) over 16,384 parameters
                  drawn like a trained run (rho in [-8, -2], log-uniform
                  gradients, Adam states with v ~ m^2), plus special values

    python tests/golden/make_golden.py posterior   # write only the named fixtures
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import Oracle  # noqa: E402
import gen  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def posterior(ref) -> dict:
    g = gen.rng(606)
    n = 16384
    mu = gen.normal(g, (n,), 0, 0.02)
    rho = (g.random(n) * 6.0 - 8.0).astype(np.float32)
    sp = gen.special_floats()
    rho = np.concatenate([rho, sp[np.isfinite(sp) & (np.abs(sp) < 100)]]).astype(np.float32)
    n = rho.size
    mu = np.concatenate([mu, gen.normal(g, (n - mu.size,), 0, 0.02)]).astype(np.float32)
    sign = np.where(g.random(n) < 0.5, -1.0, 1.0)
    dw = (sign * 10.0 ** (g.random(n) * 9.0 - 9.0)).astype(np.float32)
    eps = gen.normal(g, (n,))
    dmu0, drho0 = gen.normal(g, (n,), 0, 1e-3), gen.normal(g, (n,), 0, 1e-3)
    dmu, drho = dmu0.copy(), drho0.copy()
    ref.bayes_backward(dmu, drho, dw, eps, rho, n)
    kl = np.float64(ref.kl_forward(mu, rho, n, 0.1))
    kmu, krho = dmu0.copy(), drho0.copy()
    ref.kl_backward(kmu, krho, mu, rho, n, 0.1, 1.0 / 300000.0)
    m0 = (dw * gen.normal(g, (n,), 1.0, 0.3)).astype(np.float32)
    v0 = (m0.astype(np.float64) ** 2 * (1.0 + g.random(n))).astype(np.float32)
    adam = {}
    for t in (1, 7):
        p_, m_, v_ = mu.copy(), m0.copy(), v0.copy()
        ref.adamw_update(p_, dw, m_, v_, n, t, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        adam.update({f"p{t}": p_, f"m{t}": m_, f"v{t}": v_})
    return dict(mu=mu, rho=rho, dw=dw, eps=eps, dmu0=dmu0, drho0=drho0, dmu=dmu, drho=drho, kl=kl,
                kmu=kmu, krho=krho, m0=m0, v0=v0, **adam)


def head(ref) -> dict:
    out = {}
    for tag, (B, T, V), seed in (("s", (4, 64, 27), 707), ("l", (1, 2, 50257), 708)):
        g = gen.rng(seed)
        logits = gen.normal(g, (B, T, V), 0, 3.0)
        targets = g.integers(0, V, B * T).astype(np.int32)
        losses, probs = np.zeros(B * T, np.float32), np.zeros_like(logits)
        ref.softmax_crossentropy(losses, probs, logits, targets, B, T, V)
        d0 = gen.normal(g, (B, T, V), 0, 1e-3)
        d = d0.copy()
        ref.crossentropy_softmax_backward(d, probs, targets, B, T, V)
        out.update({f"{tag}_shape": np.array([B, T, V], np.int32), f"{tag}_logits": logits,
                    f"{tag}_targets": targets, f"{tag}_losses": losses, f"{tag}_probs": probs,
                    f"{tag}_dlogits0": d0, f"{tag}_dlogits": d})
    return out


HASHED = {"posterior": ("dmu", "drho", "kl", "kmu", "krho", "p1", "m1", "v1", "p7", "m7", "v7"),
          "head": ("s_losses", "s_probs", "s_dlogits", "l_losses", "l_probs", "l_dlogits")}


def main(only=None) -> None:
    ref = Oracle(reference=True)
    meta_path = os.path.join(HERE, "golden.json")
    digests = {}
    if only:
        with open(meta_path) as f:
            digests = json.load(f)["sha256"]
        for name in only:
            fx = {"posterior": posterior, "head": head}[name](ref)
            np.savez_compressed(os.path.join(HERE, name + ".npz"), **fx)
            digests[name] = {k: sha(fx[k]) for k in HASHED[name]}
        write_meta(meta_path, digests)
        print("wrote fixtures:", ", ".join(only))
        return

    # ---- encoder ------------------------------------------------------------
    g = gen.rng(101)
    B, T, C, V = 4, 64, 384, 27
    inp = gen.tokens_uniform(g, B * T, V)
    wte = gen.normal(g, (V, C), 0, 0.02)
    wpe = gen.normal(g, (T, C), 0, 0.01)
    dout = gen.normal(g, (B, T, C))
    dwte0 = gen.normal(g, (V, C))
    dwpe0 = gen.normal(g, (T, C))
    out = np.zeros((B, T, C), np.float32)
    ref.encoder_forward(out, inp, wte, wpe, B, T, C)
    dwte, dwpe = dwte0.copy(), dwpe0.copy()
    ref.encoder_backward(dwte, dwpe, dout, inp, B, T, C)
    # the repeated-token case
    k_inp = np.array([5, 2, 5, 0, 5, 6], np.int32)
    k_dout = gen.normal(g, (2, 3, 4))
    k_dwte = np.zeros((7, 4), np.float32)
    k_dwpe = np.zeros((3, 4), np.float32)
    ref.encoder_backward(k_dwte, k_dwpe, k_dout, k_inp, 2, 3, 4)
    enc = dict(B=B, T=T, C=C, V=V, inp=inp, wte=wte, wpe=wpe, dout=dout, dwte0=dwte0, dwpe0=dwpe0,
               out=out, dwte=dwte, dwpe=dwpe, k_inp=k_inp, k_dout=k_dout, k_dwte=k_dwte, k_dwpe=k_dwpe)
    np.savez_compressed(os.path.join(HERE, "encoder.npz"), **enc)
    digests["encoder"] = {k: sha(enc[k]) for k in ("out", "dwte", "dwpe", "k_dwte", "k_dwpe")}

    # ---- layernorm ----------------------------------------------------------
    g = gen.rng(202)
    B, T, C = 4, 64, 384
    x = gen.normal(g, (B, T, C))
    w = gen.normal(g, (C,), 1.0, 0.1)
    b = gen.normal(g, (C,), 0.0, 0.1)
    dout = gen.normal(g, (B, T, C))
    dinp0 = gen.normal(g, (B, T, C))
    dw0 = gen.normal(g, (C,))
    db0 = gen.normal(g, (C,))
    out = np.zeros_like(x)
    mean = np.zeros((B, T), np.float32)
    rstd = np.zeros((B, T), np.float32)
    ref.layernorm_forward(out, mean, rstd, x, w, b, B, T, C)
    dinp, dw, db = dinp0.copy(), dw0.copy(), db0.copy()
    ref.layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C)
    ln = dict(B=B, T=T, C=C, x=x, w=w, b=b, dout=dout, dinp0=dinp0, dw0=dw0, db0=db0, out=out, mean=mean,
              rstd=rstd, dinp=dinp, dw=dw, db=db)
    np.savez_compressed(os.path.join(HERE, "layernorm.npz"), **ln)
    digests["layernorm"] = {k: sha(ln[k]) for k in ("out", "mean", "rstd", "dinp", "dw", "db")}

    # ---- gelu ---------------------------------------------------------------
    g = gen.rng(303)
    x = np.concatenate([gen.normal(g, (65536,)), gen.special_floats(),
                        gen.normal(g, (4096,), 0, 4.0)]).astype(np.float32)
    N = x.size
    dout = gen.normal(g, (N,))
    dinp0 = gen.normal(g, (N,))
    out = np.zeros(N, np.float32)
    ref.gelu_forward(out, x, N)
    dinp = dinp0.copy()
    ref.gelu_backward(dinp, x, dout, N)
    ge = dict(x=x, dout=dout, dinp0=dinp0, out=out, dinp=dinp)
    np.savez_compressed(os.path.join(HERE, "gelu.npz"), **ge)
    digests["gelu"] = {k: sha(ge[k]) for k in ("out", "dinp")}

    # ---- residual -----------------------------------------------------------
    g = gen.rng(404)
    N = 65536
    xa = gen.normal(g, (N,))
    ya = gen.normal(g, (N,))
    dout = gen.normal(g, (N,))
    dx0 = gen.normal(g, (N,))
    dy0 = gen.normal(g, (N,))
    out = np.zeros(N, np.float32)
    ref.residual_forward(out, xa, ya, N)
    dx, dy = dx0.copy(), dy0.copy()
    ref.residual_backward(dx, dy, dout, N)
    re = dict(x=xa, y=ya, dout=dout, dx0=dx0, dy0=dy0, out=out, dx=dx, dy=dy)
    np.savez_compressed(os.path.join(HERE, "residual.npz"), **re)
    digests["residual"] = {k: sha(re[k]) for k in ("out", "dx", "dy")}

    # ---- materialize --------------------------------------------------------
    g = gen.rng(505)
    n = 65536
    mu = gen.normal(g, (n,), 0, 0.02)
    rho = gen.normal(g, (n,), -5.0, 0.1)
    eps = gen.normal(g, (n,))
    sp = gen.special_floats()
    rho = np.concatenate([rho, sp, sp, gen.normal(g, (4096,), 0, 30.0)]).astype(np.float32)
    mu = np.concatenate([mu, np.full(sp.size, 0.5, np.float32), gen.normal(g, (sp.size,)),
                         gen.normal(g, (4096,), 0, 0.02)]).astype(np.float32)
    eps = np.concatenate([eps, np.zeros(sp.size, np.float32), gen.normal(g, (sp.size,)),
                          gen.normal(g, (4096,))]).astype(np.float32)
    w = np.zeros(rho.size, np.float32)
    ref.bayes_materialize(w, mu, rho, eps, rho.size)
    ma = dict(mu=mu, rho=rho, eps=eps, w=w)
    np.savez_compressed(os.path.join(HERE, "materialize.npz"), **ma)
    digests["materialize"] = {"w": sha(w)}

    for name, make in (("posterior", posterior), ("head", head)):
        fx = make(ref)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **fx)
        digests[name] = {k: sha(fx[k]) for k in HASHED[name]}
    write_meta(meta_path, digests)
    print("wrote fixtures:", ", ".join(sorted(digests)))


def write_meta(path: str, digests: dict) -> None:
    import platform
    meta = {"generator": "tests/golden/make_golden.py",
            "reference": "train_bnn.c via make -C oracle ref (gcc -O2 -DSKIP_MAIN)",
            "glibc": platform.libc_ver()[1], "machine": platform.machine(),
            "sha256": digests}
    with open(path, "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1:] or None)
