"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The expected values come from CPU torch running the reference's op chain, not
from the oracle: the quantizers of shadowinfer/utils/quantization.py:120-178
(amax / 127 or / 7 in the input dtype, zero -> 1, round half-even, clamp), the
bucket gather and int4 row packing of shadowinfer/shadowkv/packed_kv_cache.py:
222-388 (token-major entries, gather index h*S+t, nibble q+8 high first, zero
pad on odd rows), the plan fingerprint of shadowinfer/shadowkv/
precision_plan.py:179-190, the evict compaction of packed_kv_cache.py:666-740,
apply_reuse_mask (packed_kv_cache.py:753-854, restated over dense [S, H]
maps of the previous cache's bucket and row) and INT8Linear (shadowinfer/ffn_optimizer/int8_linear.py:65-115, the int32
product as an exact int64 matmul).

Inputs come from a counter-based integer generator (splitmix64), so they are
reproducible on any numpy/torch version; fp inputs are multiples of 2^-21 in
[-4, 4) (exact in fp32), with a few rows scaled x64 as outliers.
"""

import hashlib
import json
import os
import struct

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
NAMES = ("fp32", "fp16", "int8", "int4")


def splitmix64(n, seed):
    with np.errstate(over="ignore"):
        x = np.arange(n, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15)
        x = x + np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        x = x ^ (x >> np.uint64(31))
    return x


def gen_f32(shape, seed, outlier_every=0):
    n = int(np.prod(shape))
    u = (splitmix64(n, seed) >> np.uint64(40)).astype(np.int64)  # 24 random bits
    x = ((u - (1 << 23)).astype(np.float32) * np.float32(2.0 ** -21)).reshape(shape)
    if outlier_every:
        x[..., ::outlier_every] *= np.float32(64.0)
    return x


def gen_codes(S, H, seed, choices=(0, 1, 2, 3, 4), sink=0):
    c = np.array(choices, np.int8)[(splitmix64(S * H, seed) % np.uint64(len(choices))).astype(np.int64)]
    c = c.reshape(S, H)
    c[:sink, :] = 1
    return c


def gen_uniform(n, seed):
    return ((splitmix64(n, seed) >> np.uint64(40)).astype(np.float64) / float(1 << 24))


# ------------------------------------------------------- the reference's op chain
def q_int8(t):
    s = t.abs().max(dim=-1, keepdim=True)[0] / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.round(t / s).clamp(-128, 127).to(torch.int8), s


def q_int4(t, g):
    r = t.reshape(*t.shape[:-1], t.shape[-1] // g, g)
    s = r.abs().max(dim=-1, keepdim=True)[0] / 7.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    return torch.round(r / s).clamp(-8, 7).to(torch.int8), s


def pack_int4_rows(q):
    u = (q.to(torch.int16) + 8).to(torch.uint8)
    if u.shape[1] % 2:
        u = torch.cat([u, torch.zeros(u.shape[0], 1, dtype=torch.uint8)], dim=1)
    return ((u[:, 0::2] << 4) | (u[:, 1::2] & 0xF)).reshape(-1)


def pack(k, v, codes, group):
    B, H, S, D = k.shape
    geff = group if D % group == 0 else D
    out = {}
    for p, name in enumerate(NAMES):
        ts, hs = np.nonzero(codes == p)  # row-major over [S, H]: token-major order
        if ts.size == 0:
            continue
        idx = torch.from_numpy(hs.astype(np.int64) * S + ts.astype(np.int64))
        d = {"indices": np.stack([ts, hs], 1).astype(np.int32)}
        for j, x in (("k", k), ("v", v)):
            rows = x.reshape(B, H * S, D).index_select(1, idx).permute(1, 0, 2).contiguous()
            if name == "fp32":
                d[j] = rows.to(torch.float32)
            elif name == "fp16":
                d[j] = rows.to(torch.float16)
            elif name == "int8":
                d[j], d["scale_" + j] = q_int8(rows)
            else:
                q, s = q_int4(rows, geff)
                d[j] = pack_int4_rows(q.reshape(q.shape[0], -1))
                d["scale_" + j] = s.reshape(q.shape[0] * B, D // geff, 1)
        out[name] = d
    return out


def unpack(packed, B, H, S, D, group):
    geff = group if D % group == 0 else D
    ko = torch.zeros(B, H, S, D)
    vo = torch.zeros(B, H, S, D)
    for name, d in packed.items():
        t = torch.from_numpy(d["indices"][:, 0].astype(np.int64))
        h = torch.from_numpy(d["indices"][:, 1].astype(np.int64))
        n = t.numel()
        for j, o in (("k", ko), ("v", vo)):
            if name in ("fp32", "fp16"):
                x = d[j].float()
            elif name == "int8":
                x = d[j].float() * d["scale_" + j].float()
            else:
                by = d[j].reshape(n, -1)
                nib = torch.stack([by >> 4, by & 0xF], -1).reshape(n, -1)[:, :B * D]
                q = nib.to(torch.int16) - 8
                s = d["scale_" + j].reshape(n, B, D // geff, 1).float()
                x = (q.float().reshape(n, B, D // geff, geff) * s).reshape(n, B, D)
            o[:, h, t, :] = x.permute(1, 0, 2)
    return ko, vo


def evict(packed, drop):
    """Stable compaction of every bucket without the entries in ``drop``
    (packed_kv_cache.py:679-737); returns the new buckets and the count removed."""
    out, removed = {}, 0
    for name, d in packed.items():
        keep = np.array([(int(t), int(h)) not in drop for t, h in d["indices"]], bool)
        removed += int((~keep).sum())
        if not keep.any():
            continue
        ki = torch.from_numpy(np.nonzero(keep)[0].astype(np.int64))
        n = len(keep)
        nd = {"indices": d["indices"][keep]}
        for j in ("k", "v"):
            if name == "int4":
                nd[j] = d[j].reshape(n, -1).index_select(0, ki).reshape(-1)
                s = d["scale_" + j]
                nd["scale_" + j] = s.reshape(n, -1, *s.shape[1:]).index_select(0, ki).reshape(-1, *s.shape[1:])
            else:
                nd[j] = d[j].index_select(0, ki)
                if "scale_" + j in d:
                    nd["scale_" + j] = d["scale_" + j].index_select(0, ki)
        out[name] = nd
    return out, removed


def reuse(cur, prev, mask, B):
    """apply_reuse_mask (packed_kv_cache.py:753-854) over dense [S, H] maps.

    ``pcode[t, h]`` is the bucket (0..3) that holds entry (t, h) in the
    previous cache and ``ppos[t, h]`` its row there; both are -1 where the
    previous cache holds no such entry (code 4, evicted after packing, or t at
    or beyond its seq_len). A current entry whose mask is set takes the
    previous row when the buckets agree; when the previous cache holds it in
    another bucket it is counted as skipped; otherwise nothing happens. Row
    copies are the reference's index_select + index_copy_. Returns the new
    buckets and (applied, skipped_precision)."""
    S, H = mask.shape
    pcode = np.full((S, H), -1, np.int64)
    ppos = np.full((S, H), -1, np.int64)
    for p, name in enumerate(NAMES):
        if name not in prev:
            continue
        ix = prev[name]["indices"].astype(np.int64)
        inside = ix[:, 0] < S
        pcode[ix[inside, 0], ix[inside, 1]] = p
        ppos[ix[inside, 0], ix[inside, 1]] = np.nonzero(inside)[0]
    out, applied, skipped = {}, 0, 0
    for p, name in enumerate(NAMES):
        if name not in cur:
            continue
        d = {key: (t.clone() if isinstance(t, torch.Tensor) else t.copy()) for key, t in cur[name].items()}
        out[name] = d
        ix = d["indices"].astype(np.int64)
        sel = mask[ix[:, 0], ix[:, 1]]
        pc = pcode[ix[:, 0], ix[:, 1]]
        skipped += int((sel & (pc >= 0) & (pc != p)).sum())
        tgt_np = np.nonzero(sel & (pc == p))[0]
        if tgt_np.size == 0:
            continue
        applied += int(tgt_np.size)
        tgt = torch.from_numpy(tgt_np)
        src = torch.from_numpy(ppos[ix[tgt_np, 0], ix[tgt_np, 1]])
        n, pn = len(ix), len(prev[name]["indices"])
        for j in ("k", "v"):
            if name == "int4":
                rows = d[j].reshape(n, -1)
                rows.index_copy_(0, tgt, prev[name][j].reshape(pn, -1).index_select(0, src))
                d[j] = rows.reshape(-1)
                G = d["scale_" + j].shape[1]
                sc = d["scale_" + j].reshape(n, B, G, 1)
                sc.index_copy_(0, tgt, prev[name]["scale_" + j].reshape(pn, B, G, 1).index_select(0, src))
                d["scale_" + j] = sc.reshape(n * B, G, 1)
            else:
                d[j].index_copy_(0, tgt, prev[name][j].index_select(0, src))
                if "scale_" + j in d:
                    d["scale_" + j].index_copy_(0, tgt, prev[name]["scale_" + j].index_select(0, src))
    return out, applied, skipped


def raw(t):
    """Bytes of a tensor (bf16/fp16 as uint16, the rest as numpy)."""
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def digest(t):
    return hashlib.sha256(raw(t).tobytes()).hexdigest()


def fingerprint(codes, reuse_flat):
    S, H = codes.shape
    h = hashlib.sha256(struct.pack("<QQ", S, H) + codes.astype(np.int8).tobytes()
                       + np.asarray(reuse_flat, "<i8").tobytes())
    return h.hexdigest()


# ------------------------------------------------------------------ fixtures
def kv_case(path, dtype, B, H, S, D, group, seed):
    k = torch.from_numpy(gen_f32((B, H, S, D), seed, outlier_every=29)).to(dtype)
    v = torch.from_numpy(gen_f32((B, H, S, D), seed + 1)).to(dtype)
    codes = gen_codes(S, H, seed + 2)
    packed = pack(k, v, codes, group)
    ko, vo = unpack(packed, B, H, S, D, group)
    arrays = {"k": raw(k), "v": raw(v), "codes": codes, "unpack_k": ko.numpy(),
              "unpack_v": vo.numpy()}
    for name, d in packed.items():
        for key, t in d.items():
            arrays[f"{name}.{key}"] = t if isinstance(t, np.ndarray) else raw(t)
    np.savez_compressed(path, **arrays)


def config1_digests():
    """B=1, H=8, S=512, D=64 fp32, codes uniform over {fp16, int8, int4}, rows
    0-3 fp16 (sink), int4 group 16; then evict the 25% lowest-importance
    token-heads (stable ascending order over the token-major flat index,
    sinks included)."""
    B, H, S, D, g = 1, 8, 512, 64, 16
    k = torch.from_numpy(gen_f32((B, H, S, D), 101))
    v = torch.from_numpy(gen_f32((B, H, S, D), 102))
    codes = gen_codes(S, H, 103, choices=(1, 2, 3), sink=4)
    imp = gen_uniform(S * H, 104)
    order = np.argsort(imp, kind="stable")[: (S * H) // 4]
    drop = {(int(e // H), int(e % H)) for e in order}
    packed = pack(k, v, codes, g)
    ko, vo = unpack(packed, B, H, S, D, g)
    ev, removed = evict(packed, drop)
    evk, evv = unpack(ev, B, H, S, D, g)

    def bucket_digests(p):
        return {f"{name}.{key}": digest(t) for name, d in p.items() for key, t in d.items()
                if key != "indices"}

    reuse = sorted(e for e in range(S * H) if gen_uniform(S * H, 105)[e] < 0.5)
    reuse_flat = [(e % H) * S + e // H for e in reuse]
    mem = sum(raw(t).nbytes for d in packed.values() for key, t in d.items() if key != "indices")
    return {
        "shape": [B, H, S, D], "group": g, "seeds": {"k": 101, "v": 102, "codes": 103,
                                                    "importance": 104, "reuse": 105},
        "codes_sha256": hashlib.sha256(codes.tobytes()).hexdigest(),
        "buckets": bucket_digests(packed),
        "counts": {n: int(len(d["indices"])) for n, d in packed.items()},
        "memory_bytes": int(mem),
        "unpack_k": digest(ko), "unpack_v": digest(vo),
        "evict_removed": removed,
        "evict_buckets": bucket_digests(ev),
        "evict_unpack_k": digest(evk), "evict_unpack_v": digest(evv),
        "fingerprint_no_reuse": fingerprint(codes, []),
        "fingerprint_reuse": fingerprint(codes, reuse_flat),
    }


def reuse_case(path, B=2, H=4, S=24, S_prev=16, D=32, group=16, seed=400):
    """apply_reuse_mask from a previous cache that is shorter (S_prev < S),
    holds evicted entries (code 4, and entries evicted after packing) and puts
    many entries in other buckets than the current cache, bf16 K/V. The mask
    sets about 60% of the current token-heads, the rest are False."""
    dt = torch.bfloat16
    k = torch.from_numpy(gen_f32((B, H, S, D), seed, outlier_every=13)).to(dt)
    v = torch.from_numpy(gen_f32((B, H, S, D), seed + 1)).to(dt)
    kp = torch.from_numpy(gen_f32((B, H, S_prev, D), seed + 2, outlier_every=7)).to(dt)
    vp = torch.from_numpy(gen_f32((B, H, S_prev, D), seed + 3)).to(dt)
    codes = gen_codes(S, H, seed + 4)
    # the previous step's codes: the current ones with about 40% redrawn
    codes_prev = codes[:S_prev].copy()
    redraw = gen_uniform(S_prev * H, seed + 8).reshape(S_prev, H) < 0.4
    codes_prev[redraw] = gen_codes(S_prev, H, seed + 5)[redraw]
    cur = pack(k, v, codes, group)
    prev = pack(kp, vp, codes_prev, group)
    present = [(int(t), int(h)) for t, h in zip(*np.nonzero(codes_prev != 4))]
    pick = gen_uniform(len(present), seed + 6) < 0.2
    drop = sorted(e for e, x in zip(present, pick) if x)
    prev, removed = evict(prev, set(drop))
    assert removed == len(drop)
    mask = gen_uniform(S * H, seed + 7).reshape(S, H) < 0.6
    out, applied, skipped = reuse(cur, prev, mask, B)
    ko, vo = unpack(out, B, H, S, D, group)
    arrays = {"k": raw(k), "v": raw(v), "k_prev": raw(kp), "v_prev": raw(vp), "codes": codes,
              "codes_prev": codes_prev, "drop": np.array(drop, np.int32).reshape(-1, 2),
              "mask": mask, "applied": np.int64(applied), "skipped_precision": np.int64(skipped),
              "unpack_k": ko.numpy(), "unpack_v": vo.numpy()}
    for name, d in out.items():
        for key, t in d.items():
            arrays[f"{name}.{key}"] = t if isinstance(t, np.ndarray) else raw(t)
    np.savez_compressed(path, **arrays)


def int8_linear_case(path, M=8, K=128, N=96, seed=300):
    w = torch.from_numpy(gen_f32((N, K), seed)) * 0.005
    x = torch.from_numpy(gen_f32((M, K), seed + 1)).to(torch.bfloat16)
    bias = torch.from_numpy(gen_f32((N,), seed + 2)) * 0.01
    sw = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    qw = torch.clamp(torch.round(w / sw[:, None]), -127, 127).to(torch.int8)  # [N, K]
    xf = x.float()
    sx = (xf.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    qx = torch.clamp(torch.round(xf / sx[:, None]), -127, 127).to(torch.int8)
    acc = (qx.to(torch.int64) @ qw.t().to(torch.int64)).to(torch.int32)
    scale = sx[:, None] * sw[None, :]
    out = (acc.float() * scale).to(x.dtype)
    out_b = (acc.float() * scale + bias).to(x.dtype)
    np.savez_compressed(path, w=w.numpy(), x=raw(x), bias=bias.numpy(), qweight_kn=qw.t().contiguous().numpy(),
                        weight_scale=sw.numpy(), act_q=qx.numpy(), act_scale=sx.numpy(),
                        acc=acc.numpy(), out=raw(out), out_bias=raw(out_b))


def main():
    kv_case(os.path.join(HERE, "kv_f32_b1h4s24d64.npz"), torch.float32, 1, 4, 24, 64, 16, 11)
    kv_case(os.path.join(HERE, "kv_bf16_b2h3s17d48.npz"), torch.bfloat16, 2, 3, 17, 48, 16, 21)
    kv_case(os.path.join(HERE, "kv_bf16_b1h2s9d45.npz"), torch.bfloat16, 1, 2, 9, 45, 16, 31)
    int8_linear_case(os.path.join(HERE, "int8_linear_m8k128n96.npz"))
    reuse_case(os.path.join(HERE, "reuse_bf16_b2h4s24p16d32.npz"))
    with open(os.path.join(HERE, "config1_digests.json"), "w") as f:
        json.dump(config1_digests(), f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
