"""Write ``metadata_fixtures.json``: input/output vectors of the reference
metadata scheduler (sparse_attn_sharedkv_tilelang/metadata.py:1018-1086).

Runs only in the build container, where the reference tree is mounted; the
committed JSON is the fixture, the reference never travels. The scheduler is
integer-only and its only other pins are one worked example and a few
invariants, so its outputs on arbitrary inputs are recorded here.

Each case stores the keyword arguments (tensors as int lists) and the
non-zero entries of the int32[1024] output as ``[index, value]`` pairs.

    python tests/golden/make_metadata_fixtures.py
"""

from __future__ import annotations

import json
import os
import random
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference/sparse_attn_sharedkv_tilelang"


def _kw_to_json(kw):
    out = {}
    for k, v in kw.items():
        out[k] = v.tolist() if isinstance(v, torch.Tensor) else v
    return out


def _kw_from_json(kw):
    out = dict(kw)
    for k in ("cu_seqlens_q", "cu_seqlens_ori_kv", "cu_seqlens_cmp_kv", "seqused_q", "seqused_kv"):
        if out.get(k) is not None:
            out[k] = torch.tensor(out[k], dtype=torch.int32)
    return out


def cases():
    sys.path.insert(0, REPO)
    from dsv4_amd import cases as C

    out = []
    # Worked example of the reference design note (B=2, aic=3, SCFA r=128).
    out.append(("kat_doc_b2_aic3", dict(
        num_heads_q=64, num_heads_kv=1, head_dim=512,
        cu_seqlens_q=torch.tensor([0, 4, 6], dtype=torch.int32),
        seqused_kv=torch.tensor([1500, 500], dtype=torch.int32),
        batch_size=2, max_seqlen_q=4, max_seqlen_kv=1500, cmp_topk=512, cmp_ratio=128,
        layout_q="TND", aic_core_num=3, aiv_core_num=6)))
    # The reference suite's six scenarios.
    for name, cfg in C.REF_SCENARIOS.items():
        ql, kl = C.seq_lengths(cfg)
        kw = dict(num_heads_q=cfg.H, num_heads_kv=1, head_dim=cfg.D,
                  cu_seqlens_q=torch.tensor([0, ql[0]], dtype=torch.int32),
                  seqused_kv=torch.tensor(kl, dtype=torch.int32), batch_size=1,
                  max_seqlen_q=ql[0], max_seqlen_kv=max(kl), layout_q="TND",
                  has_cmp_kv=cfg.scenario >= 2)
        if cfg.scenario >= 2:
            kw["cmp_ratio"] = cfg.cmp_ratio
        if cfg.scenario == 3:
            kw["cmp_topk"] = cfg.K
        out.append((f"ref_{name}", kw))
    # The five measured workloads, with the exact seeded lengths.
    for name, cfg in C.CONFIGS.items():
        ql, kl = C.seq_lengths(cfg)
        cu = [0]
        for x in ql:
            cu.append(cu[-1] + x)
        out.append((f"cfg_{name}", dict(
            num_heads_q=cfg.H, num_heads_kv=1, head_dim=cfg.D,
            cu_seqlens_q=torch.tensor(cu, dtype=torch.int32),
            seqused_kv=torch.tensor(kl, dtype=torch.int32), batch_size=cfg.B,
            max_seqlen_q=max(ql), max_seqlen_kv=max(kl), cmp_topk=cfg.K,
            cmp_ratio=cfg.cmp_ratio, layout_q="TND")))
    # Random fuzz over layouts, scenarios, head counts, core counts, masks.
    rnd = random.Random(1234)
    for i in range(60):
        B = rnd.choice([1, 2, 3, 5, 8, 16, 32, 64])
        layout = rnd.choice(["TND", "TND", "BSND"])
        n2 = rnd.choice([1, 1, 1, 2])
        g = rnd.choice([16, 64, 128])
        scen = rnd.choice([1, 2, 3, 3])
        ratio = rnd.choice([4, 4, 128])
        ql = [rnd.choice([0, 1, 1, 2, 3, 4, 7, 33, 300]) for _ in range(B)]
        if rnd.random() < 0.3:
            ql = [rnd.choice([1, 2, 4])] * B
        kl = [max(0, q + rnd.choice([0, 1, 5, 100, 1000, 5000, 20000]) -
                  rnd.choice([0, 0, 0, 3])) for q in ql]
        kw = dict(num_heads_q=g * n2, num_heads_kv=n2, head_dim=rnd.choice([512, 576]),
                  seqused_kv=torch.tensor(kl, dtype=torch.int32), batch_size=B,
                  max_seqlen_q=max(ql), max_seqlen_kv=max(kl) if kl else 0,
                  layout_q=layout, has_cmp_kv=scen >= 2,
                  aic_core_num=rnd.choice([24, 24, 36, 8, 3, 1]),
                  aiv_core_num=rnd.choice([48, 72, 6]),
                  ori_win_left=rnd.choice([127, 127, 63, 0, -1]),
                  ori_mask_mode=rnd.choice([4, 4, 4, 3, 0]))
        if layout == "TND":
            cu = [0]
            for x in ql:
                cu.append(cu[-1] + x)
            kw["cu_seqlens_q"] = torch.tensor(cu, dtype=torch.int32)
        elif rnd.random() < 0.5:
            kw["seqused_q"] = torch.tensor(ql, dtype=torch.int32)
        if scen >= 2:
            kw["cmp_ratio"] = ratio
        if scen == 3:
            kw["cmp_topk"] = rnd.choice([64, 512, 1024])
        out.append((f"fuzz_{i:02d}", kw))
    return out


def main():
    sys.path.insert(0, REF)
    import metadata as refmd  # reference scheduler, this container only

    import signal

    def _alarm(signum, frame):
        raise TimeoutError

    signal.signal(signal.SIGALRM, _alarm)
    records = []
    for name, kw in cases():
        signal.alarm(20)
        try:
            md = refmd.sparse_attn_sharedkv_metadata(**kw)
        except TimeoutError:
            print(f"{name}: reference scheduler did not finish in 20 s; case dropped")
            continue
        finally:
            signal.alarm(0)
        nz = [[int(i), int(v)] for i, v in enumerate(md.tolist()) if v != 0]
        records.append(dict(name=name, kwargs=_kw_to_json(kw), nonzero=nz))
    path = os.path.join(HERE, "metadata_fixtures.json")
    with open(path, "w") as f:
        json.dump(dict(source="sparse_attn_sharedkv_tilelang/metadata.py", size=1024,
                       cases=records), f, separators=(",", ":"))
    print(f"wrote {len(records)} cases to {path}")


if __name__ == "__main__":
    main()
