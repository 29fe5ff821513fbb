"""Write golden vectors of the reference NSAAttention 'ref' path.

Run once, in the build container, with the reference checkout at
/root/reference (read-only; nothing of it is copied):

    python tests/golden/make_nsa_model_golden.py [/root/reference]

For every config of model_params.CONFIGS it builds the reference's
``NSAAttention(attn_impl='ref')`` (nsa_model.py:130-304) in float64 on the CPU,
sets its parameters with model_params.init_params, runs forward and backward
on model_params.inputs, and stores the output, the input and parameter
gradients (rounded to float32) and the block indices its ``torch.topk``
returned (nsa_model.py:258), in ``nsa_model_golden.npz`` beside this script.
For every config of model_params.MODEL_CONFIGS it does the same for the
reference's ``NSATransformer`` (nsa_model.py:455-511): logits, loss, parameter
gradients, each layer's top-k indices, the state_dict layout and
``num_params()``.  The inputs are regenerated from their seed by the tests;
their float64 sums are stored to check that.  Those indices are the one thing
no closed form pins: the order ``torch.topk`` gives to tied scores.
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import model_params  # noqa: E402


def main(ref_dir):
    sys.path.insert(0, ref_dir)
    import nsa_model as ref  # the reference module, CPU only

    out = {}
    meta = []
    for name, cfg, B, T in model_params.CONFIGS:
        m = ref.NSAAttention(**cfg, attn_impl="ref").double()
        model_params.init_params(m, seed=1)
        x, dy = model_params.inputs(cfg, B, T, seed=2)
        x.requires_grad_()
        seen = []
        topk = torch.topk

        def recording_topk(*a, **k):
            r = topk(*a, **k)
            seen.append(r.indices.detach().clone())
            return r

        torch.topk = recording_topk
        try:
            y = m(x)
        finally:
            torch.topk = topk
        y.backward(dy)
        assert len(seen) == 1, "expected one top-k call per forward"
        out[f"{name}/input_sums"] = np.array([float(x.detach().sum()), float(dy.sum())])
        out[f"{name}/y"] = y.detach().numpy().astype(np.float32)
        out[f"{name}/dx"] = x.grad.numpy().astype(np.float32)
        out[f"{name}/topk"] = seen[0].numpy().astype(np.int32)
        for pname, p in sorted(m.named_parameters()):
            out[f"{name}/grad/{pname}"] = p.grad.numpy().astype(np.float32)
        meta.append(dict(name=name, cfg=cfg, B=B, T=T))
    # the model around the layer (nsa_model.py:377-556): logits, loss, every
    # parameter gradient, the state_dict layout and each layer's top-k
    model_meta = []
    for name, cfg, B, T in model_params.MODEL_CONFIGS:
        m = ref.NSATransformer(**cfg, attn_impl="ref").double()
        model_params.init_params(m, seed=3)
        x, y = model_params.tokens(cfg, B, T, seed=4)
        seen = []
        topk = torch.topk

        def recording_topk(*a, **k):
            r = topk(*a, **k)
            seen.append(r.indices.detach().clone())
            return r

        torch.topk = recording_topk
        try:
            logits, loss = m(x, y)
        finally:
            torch.topk = topk
        loss.backward()
        out[f"{name}/logits"] = logits.detach().numpy().astype(np.float32)
        out[f"{name}/loss"] = np.array([float(loss)])
        for i, ix in enumerate(seen):
            out[f"{name}/topk{i}"] = ix.numpy().astype(np.int32)
        for pname, p in sorted(m.named_parameters()):
            out[f"{name}/grad/{pname}"] = p.grad.numpy().astype(np.float32)
        layout = {k: list(v.shape) for k, v in m.state_dict().items()}
        model_meta.append(dict(name=name, cfg=cfg, B=B, T=T, n_topk=len(seen), state_dict=layout,
                               num_params=int(m.num_params())))
    out["model_meta"] = np.frombuffer(json.dumps(model_meta).encode(), dtype=np.uint8)
    out["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, "nsa_model_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
