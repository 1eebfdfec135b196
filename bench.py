"""WKV7 benchmark on one MI355X.

Default workload: WKV7 forward (saving the state every 16
steps) + backward, B=4, T=2048, H=80, N=64, bf16 I/O, fp32 state, s0 ~
N(0,0.1), dsT = 0, synthetic inputs resident in HBM.  One step = one forward
and one backward over the batch, through the C ABI (theseus.wkv7.extension()).

Prints ONE JSON line: tokens/s, achieved algorithmic HBM GB/s of the whole
fwd+bwd and, as ``roofline``, that of the dominant kernel timed with HIP
events on the stream the kernels run on; ``cpu_baseline`` times the
reference's PyTorch op sequence (float32, autograd) on the host cores over a
bounded slice of the same workload.

Counted traffic (``roofline.traffic``, ``hbm_frac_counted``) is not measured in
this run: it is the per-launch FETCH_SIZE + WRITE_SIZE of committed rocprofv3
--pmc runs (profiles/wkv7_<config>_traffic.json, source named in the line).  At
config 2 it is the algorithmic bytes plus the saved states the config mandates
(a state every 16 steps, written by the forward and read by the backward,
0.676 GB each way), 3.075 GB per step: even at the full 8 TB/s a step takes
0.384 ms, which caps the algorithmic fraction near 55 %.

Other configurations (``--config``): c1 = 8 chained T=512 forward calls without
saved states (state carried), B=1, H=80, with one T=4096 call timed beside them (both
on the time-split forward: 80 heads leave CUs for 3 segments per head); c4 = 256 in-place decode steps at
B=64, with one fused T=256 forward timed beside them; c3 = the TimeMix layer;
c4tm = config 4 through a whole TimeMix layer (C=5120, bf16 serving weights): 256
tokens per step, served out of place (the reference's T=1 forward), in place
(TimeMix.step_) and as a captured HIP graph of the in-place step (the timed one);
optim = the optimizer step after backward over one C=5120 TimeMix layer's 112 M
float32 parameters (gradient scale, clip_grad_norm_, AdamW), fused
(theseus.optim.FusedAdamW) against the reference's torch sequence; gdn = the teacher's
gated delta rule (Qwen3.5 GDN geometry: 32 value heads, K = V = 128) through the WKV7
kernels' exp-decay mode (theseus.gdn), forward and forward+backward, against
transformers' torch_chunk_gated_delta_rule on the same GPU; n128 = config 2's training
step at head size 128 (B=4, T=2048, H=32: a 4096-wide layer), on the chunk-record kernels,
with one step on the step-serial kernels timed beside it.

Algorithmic bytes (compulsory contract I/O; E = H*N, S_l = H*N*N*4 bytes):
  forward  = B*T*E*2*7  + 2*B*S_l   (r,w,k,v,a,b in, y out; s0 in, sT out)
  backward = B*T*E*2*13 + 3*B*S_l   (r..b, dy in; six grads out; s0, dsT in, ds0 out)
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "rwkv-theseus_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "WKV7 fwd+bwd tokens/s (H=80,N=64,bf16) + achieved HBM GB/s as % of peak"
HBM_PEAK_GBPS = 8000.0

CONFIGS = {
    # name: B, T, H, N, s0_std, seed
    "c2": dict(B=4, T=2048, H=80, N=64, s0_std=0.1, seed=20262),
    "c1": dict(B=1, T=4096, H=80, N=64, s0_std=0.0, seed=20261),
    "c4": dict(B=64, T=256, H=80, N=64, s0_std=0.0, seed=20264),
    "c3": dict(B=2, T=4096, H=80, N=64, s0_std=0.0, seed=20263),
    "c4tm": dict(B=64, T=256, H=80, N=64, s0_std=0.0, seed=20264),
    "optim": dict(B=0, T=0, H=80, N=64, s0_std=0.0, seed=20265),
    "gdn": dict(B=1, T=2048, H=32, N=128, s0_std=0.0, seed=20266),
    "n128": dict(B=4, T=2048, H=32, N=128, s0_std=0.1, seed=20267),
}


def timemix_step_flops(B, T, C, rank, grank):
    """Matrix FLOPs of one TimeMix forward+backward: 4 dense CxC projections and the
    w/a (rank) and g (grank) LoRAs, each 2*M*K*N forward and twice that backward."""
    M = B * T
    fwd = 4 * 2 * M * C * C + 2 * (2 * 2 * M * C * rank) + 2 * 2 * M * C * grank
    return 3 * fwd


def bench_timemix(args, cfg):
    """Config 3: one TimeMix layer (C=5120, H=80, N=64, reference geometry: w/a LoRA rank 192,
    g rank 352, no v-LoRA) forward+backward, bf16 autocast over fp32 parameters, weights
    N(0,0.02), x ~ N(0,1)."""
    import torch
    from theseus.timemix import TimeMix

    B, T, H, N = cfg["B"], cfg["T"], cfg["H"], cfg["N"]
    C = H * N
    torch.manual_seed(cfg["seed"])
    m = TimeMix(C, 3, 8, head_size=N, backend="cuda").cuda()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 2 and name != "r_k":
                p.normal_(0, .02)
    if args.timemix_unfused:
        import theseus.fused as fz
        fz.available = lambda *a, **k: False
    x = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16)
    gy = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16)

    def one_step():
        m.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, _ = m(x)
        y.backward(gy)

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    rank = max(32, round(2.5 * (C ** .5) / 32) * 32)
    grank = max(32, round(5 * (C ** .5) / 32) * 32)
    fl = timemix_step_flops(B, T, C, rank, grank)
    tflops = fl / (ms * 1e-3) / 1e12
    print(json.dumps({
        "metric": "TimeMix layer fwd+bwd tokens/s (C=5120, H=80, N=64, bf16 autocast)",
        "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "timemix_fwd_bwd", "B": B, "T": T, "C": C, "lora_rank": rank,
                   "gate_rank": grank, "fused_elementwise": not args.timemix_unfused},
        "roofline": {"kernel": "layer (GEMM-dominated)", "bound": "mfma", "achieved": round(tflops, 1),
                     "peak": 2500.0, "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4), "traffic": None}}),
        flush=True)


def bench_serving(args, cfg):
    """Config 4 through a TimeMix layer: B=64 lanes, 256 consecutive tokens, one per call,
    C=5120 (H=80, N=64), bf16 weights as the reference's install() loads a layer for
    inference (hf_model.py:147-148), weights N(0,0.02), x ~ N(0,1).  Three ways of serving
    a token: the out-of-place T=1 forward (what the reference's Runner calls), the in-place
    TimeMix.step_, and a HIP graph of step_ (theseus.serving.CapturedStep) -- the timed
    step replays the graph 256 times.  Per-token HBM bytes: the layer's bf16 weights once
    plus the fp32 WKV state read and written (2*B*S_l) plus activations."""
    import torch
    from theseus import fused
    from theseus.serving import CapturedStep, serving_state
    from theseus.timemix import TimeMix

    B, T, H, N = cfg["B"], cfg["T"], cfg["H"], cfg["N"]
    C = H * N
    torch.manual_seed(cfg["seed"])
    m = TimeMix(C, 3, 8, head_size=N, backend="cuda")
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 2 and name != "r_k":
                p.normal_(0, .02)
    m = m.cuda().to(torch.bfloat16).eval()
    x = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16)
    toks = [x[:, t:t + 1].contiguous() for t in range(T)]
    st0 = m.initial_state(x)
    st_ip = serving_state(st0)
    graph = CapturedStep(m, serving_state(st0), toks[0], autocast=None)

    # the eager modes run as a serving loop that keeps the layer's derived parameter copies
    # (float32 vectors, stacked lerp coefficients, transposed LoRAs) in a store of its own,
    # as the captured graph does (theseus.fused.param_cache); inside it each step is one
    # native call (theseus_tm_serving_step)
    store = {}

    def run(mode):
        if mode == "out_of_place":
            st = st0
            with fused.param_cache(store):
                for t in range(T):
                    _, st = m(toks[t], st)
        elif mode == "in_place":
            with fused.param_cache(store):
                for t in range(T):
                    m.step_(toks[t], st_ip)
        else:
            for t in range(T):
                graph(toks[t])

    per_token = {}
    modes = [md for md in args.serving_modes.split(",") if md]
    with torch.no_grad():
        for mode in modes:
            for _ in range(max(1, args.warmup // 5)):
                run(mode)
            torch.cuda.synchronize()
            n = max(1, args.steps // 10) if mode != "graph" else max(1, args.steps // 5)
            t0 = time.perf_counter()
            for _ in range(n):
                run(mode)
            torch.cuda.synchronize()
            per_token[mode] = (time.perf_counter() - t0) * 1e3 / (n * T)
    ms_tok = per_token["graph"] if "graph" in per_token else min(per_token.values())
    weight_bytes = sum(p.numel() * p.element_size() for p in m.parameters())
    state_bytes = 2 * B * H * N * N * 4
    act_bytes = B * C * 2 * 8  # x in, out, and the mixes / WKV operands that stay small at T=1
    step_bytes = weight_bytes + state_bytes + act_bytes
    gbps = step_bytes / (ms_tok * 1e-3) / 1e9
    print(json.dumps({
        "metric": "TimeMix serving step tokens/s (config 4 through the layer, C=5120, B=64)",
        "value": round(B / (ms_tok * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": max(1, args.steps // 5), "warmup": max(1, args.warmup // 5),
        "ms_per_step": round(ms_tok * T, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "timemix_serving_step", "B": B, "tokens_per_step": T, "C": C, "H": H,
                   "N": N, "weights": "bf16", "state_dtype": "fp32"},
        "ms_per_token": {k: round(v, 4) for k, v in per_token.items()},
        "roofline": {"kernel": "whole serving step (graph replay)", "bound": "hbm",
                     "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "alg_bytes_per_launch": step_bytes}}), flush=True)


def bench_optim(args, cfg):
    """The step after backward (train.py:202-208) over a C=5120 TimeMix layer's parameter
    schema (112,460,800 float32 parameters in 23 tensors, theseus/stage.py:36-42 groups),
    gradients ~N(0, 1e-4) with scale 0.5 and clip norm 1.0 (so the clip is active).  One
    step of FusedAdamW.step_after_backward against the reference's p.grad.mul_ loop +
    clip_grad_norm_(error_if_nonfinite=True) + torch.optim.AdamW(fused=True).step(), each
    timed with HIP events on the current stream.  Algorithmic bytes per parameter: read
    param, grad and both moments, write param and moments (28 B)."""
    import torch
    from theseus.optim import FusedAdamW
    from theseus.timemix import TimeMix

    C = cfg["H"] * cfg["N"]
    with torch.device("meta"):
        shapes = [p.shape for p in TimeMix(C, 3, 8, head_size=cfg["N"], backend="cuda").parameters()]
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"])

    def make():
        ps = [torch.nn.Parameter(torch.randn(sh, generator=gen, device="cuda") * .02) for sh in shapes]
        return ps, [p for p in ps if p.ndim == 2], [p for p in ps if p.ndim != 2]

    ours_p, od, on = make()
    ref_p, rd, rn = make()
    ours = FusedAdamW([{"params": od, "weight_decay": .1}, {"params": on, "weight_decay": 0.}], lr=1e-4,
                      betas=(.9, .95), eps=1e-8)
    ref = torch.optim.AdamW([{"params": rd, "weight_decay": .1}, {"params": rn, "weight_decay": 0.}], lr=1e-4,
                            betas=(.9, .95), eps=1e-8, fused=True)
    grads = [torch.randn(sh, generator=gen, device="cuda") * 1e-4 for sh in shapes]
    for p, q, g in zip(ours_p, ref_p, grads):
        p.grad, q.grad = g, g.clone()
    n_param = sum(p.numel() for p in ours_p)
    stream = torch.cuda.current_stream()

    def ours_step():
        ours.step_after_backward(grad_scale=.5, max_norm=1.0, error_if_nonfinite=True)

    def ref_step():
        for p in ref_p:
            p.grad.mul_(.5)
        torch.nn.utils.clip_grad_norm_(ref_p, 1.0, error_if_nonfinite=True)
        ref.step()

    times = {}
    for name, fn in (("fused", ours_step), ("reference_torch", ref_step)):
        for _ in range(max(2, args.warmup)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        times[name] = e0.elapsed_time(e1) / args.steps
    ms = times["fused"]
    alg = 28 * n_param
    gbps = alg / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "optimizer step after backward, parameters/s (one C=5120 TimeMix layer, fp32 AdamW + clip)",
        "value": round(n_param / (ms * 1e-3), 1), "unit": "parameters/s", "n_gpus": 1, "steps": args.steps,
        "warmup": max(2, args.warmup), "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "adamw_clip_step", "parameters": n_param, "tensors": len(shapes),
                   "grad_scale": .5, "max_norm": 1.0},
        "ms_per_step_by_impl": {k: round(v, 4) for k, v in times.items()},
        "speedup_vs_reference_torch": round(times["reference_torch"] / ms, 3),
        "roofline": {"kernel": "fused step (3 launches)", "bound": "hbm", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": 32 * n_param, "traffic_source": "by construction: gradients read twice",
                     "alg_bytes_per_launch": alg}}), flush=True)


def bench_gdn(args, cfg):
    """GDN forward (no grad) and forward+backward at B=1, T=2048, H=32, K=V=128, bf16 q/k/v
    with the layers' in-kernel q/k L2 norm, through theseus.gdn: the forward on the chunked
    MFMA kernels (theseus_gdn_forward: gdn_prep, gdn_scan), forward+backward on the chunked
    kernels too (theseus_gdn_forward_train with saved states, theseus_gdn_backward:
    gdn_bwd_prep, wkv7_bwd_scan, gdn_bwd_chunk; float32 operands as transformers computes);
    beside transformers' torch_chunk_gated_delta_rule (its torch fallback, the function the
    reference's teacher runs without FLA) and the step-serial forward of the same call."""
    import inspect

    import torch
    from theseus import gdn
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M

    B, T, H, N = cfg["B"], cfg["T"], cfg["H"], cfg["N"]
    g = torch.Generator(device="cuda").manual_seed(cfg["seed"])
    q, k, v = (torch.randn(B, T, H, N, generator=g, device="cuda").to(torch.bfloat16) for _ in range(3))
    gg = -torch.exp(torch.randn(B, T, H, generator=g, device="cuda"))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device="cuda"))
    s0 = .1 * torch.randn(B, H, N, N, generator=g, device="cuda")
    hf_chunk = inspect.unwrap(M.torch_chunk_gated_delta_rule)

    def timed(fn, n):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    def ours_fwd():
        with torch.no_grad():
            gdn.chunk_gated_delta_rule(q, k, v, gg, beta, initial_state=s0, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)

    xs = [t.detach().clone().requires_grad_() for t in (q, k, v, gg, beta, s0)]

    def ours_fwd_bwd():
        o, st = gdn.chunk_gated_delta_rule(*xs[:5], initial_state=xs[5], output_final_state=True,
                                           use_qk_l2norm_in_kernel=True)
        (o.float().sum() + st.sum()).backward()

    def hf_fwd():
        with torch.no_grad():
            hf_chunk(q, k, v, gg, beta, initial_state=s0, output_final_state=True, use_qk_l2norm_in_kernel=True)

    xh = [t.detach().clone().requires_grad_() for t in (q, k, v, gg, beta, s0)]

    def hf_fwd_bwd():
        o, st = hf_chunk(*xh[:5], initial_state=xh[5], output_final_state=True, use_qk_l2norm_in_kernel=True)
        (o.float().sum() + st.sum()).backward()

    # the kernels alone (the drop-in's own call: bf16 q/k/v, in-kernel q/k norm), and the
    # same forward on the step-serial WKV7 kernels (the path used before the chunked one)
    from theseus import wkv7 as W
    qn, kn = (gdn.l2norm(x).float().contiguous() for x in (q, k))
    vf, gf, bf = v.float().contiguous(), gg.float().contiguous(), beta.float().contiguous()
    ext = W.extension()
    st = torch.cuda.current_stream()

    def kernels_ms(n_rep):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ext.gdn_forward(q, k, v, gf, bf, s0, qk_l2norm=True)
        torch.cuda.synchronize()
        ev[0].record(st)
        for _ in range(n_rep):
            ext.gdn_forward(q, k, v, gf, bf, s0, qk_l2norm=True)
        ev[1].record(st)
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / n_rep

    def serial_fwd():
        with torch.no_grad():
            W.wkv7_ex(qn * N ** -0.5, gf.unsqueeze(-1).expand(B, T, H, N).contiguous(), kn,
                      vf * bf.unsqueeze(-1), kn, -(torch.exp(gf) * bf).unsqueeze(-1) * kn, s0,
                      flags=W.DECAY_EXP | W.STATE_KEY_VALUE)

    n = max(2, args.steps // 10)
    ms = {"ours_fwd": timed(ours_fwd, n), "ours_fwd_kernels": kernels_ms(n), "ours_fwd_bwd": timed(ours_fwd_bwd, n),
          "step_serial_fwd": timed(serial_fwd, max(1, n // 2)),
          "transformers_torch_chunk_fwd": timed(hf_fwd, max(1, n // 2)),
          "transformers_torch_chunk_fwd_bwd": timed(hf_fwd_bwd, max(1, n // 2))}
    # compulsory bytes of the two kernels: q, k, v in and o out (bf16), g, beta in (fp32),
    # state in and out (fp32); the per-chunk operands they pass through the workspace are
    # not counted
    fwd_bytes = B * T * H * N * 2 * 4 + B * T * H * 4 * 2 + 2 * B * H * N * N * 4
    gbps = fwd_bytes / (ms["ours_fwd_kernels"] * 1e-3) / 1e9
    print(json.dumps({
        "metric": "GDN (gated delta rule) forward tokens/s, Qwen3.5 GDN geometry (H=32, K=V=128)",
        "value": round(B * T / (ms["ours_fwd"] * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": n,
        "warmup": 2, "ms_per_step": round(ms["ours_fwd"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 I/O, fp32 compute", "data": "synthetic",
        "config": {"workload": "gdn_forward", "B": B, "T": T, "H": H, "K": N, "V": N,
                   "kernels": "forward: chunked MFMA GDN (gdn_prep + gdn_scan); fwd+bwd: the same with saved "
                              "states, then gdn_bwd_prep + wkv7_bwd_scan + gdn_bwd_chunk (float32 operands)"},
        "ms_by_impl": {k2: round(v2, 4) for k2, v2 in ms.items()},
        "speedup_vs_transformers_torch_chunk": round(ms["transformers_torch_chunk_fwd"] / ms["ours_fwd"], 2),
        "speedup_fwd_bwd_vs_transformers_torch_chunk": round(ms["transformers_torch_chunk_fwd_bwd"] /
                                                             ms["ours_fwd_bwd"], 2),
        "roofline": {"kernel": "forward", "bound": "latency (chunk-to-chunk chain)", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": None, "alg_bytes_per_launch": fwd_bytes}}), flush=True)


def alg_bytes(B, T, H, N, which):
    E, Sl = H * N, H * N * N * 4
    if which == "fwd":
        return B * T * E * 2 * 7 + 2 * B * Sl
    if which == "bwd":
        return B * T * E * 2 * 13 + 3 * B * Sl
    if which == "decode":  # one T=1 step over B lanes
        return B * E * 2 * 7 + 2 * B * Sl
    raise ValueError(which)


def cpu_baseline(B, H, N, T_slice, seed, budget_s=12.0, T_total=2048):
    """Reference op sequence (oracle.reference_torch = theseus/wkv7.py:16-28 restated),
    float32 autograd fwd+bwd on the host cores, over consecutive T_slice-step slices
    of the workload (state carried, detached between slices, as TimeMix training
    carries it between chunks) until ``budget_s`` seconds or T_total steps."""
    import torch
    from oracle import wkv7_oracle as O
    from theseus.synthetic import wkv7_inputs

    cores = O.cpu_count()
    torch.set_num_threads(cores)
    dt, steps, state = 0.0, 0, None
    while steps < T_total and dt < budget_s:
        inp = wkv7_inputs(B, T_slice, H, N, seed=seed + steps, dtype=torch.float32, s0_std=0.1)
        xs = [inp[n].clone().requires_grad_() for n in "rwkvab"]
        s0 = (inp["s0"] if state is None else state).clone().requires_grad_()
        t0 = time.perf_counter()
        y, sT = O.reference_torch(*xs, s0)
        torch.autograd.backward((y, sT), (inp["dy"], torch.zeros_like(sT)))
        dt += time.perf_counter() - t0
        state = sT.detach()
        steps += T_slice
    return {"value": round(B * steps / dt, 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"B={B} H={H} N={N}: {steps // T_slice} consecutive T={T_slice} slices ({steps} steps) "
                      f"of the workload, fp32 torch autograd fwd+bwd of the reference op sequence, "
                      f"{dt:.1f} s on {O.cpu_model()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="untimed steps after the warmup steps until this much time under load has "
                         "passed, before the timed steps (the GPU's clock transient)")
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-slice", type=int, default=256, help="T of each CPU baseline slice (0: skip)")
    ap.add_argument("--timemix-unfused", action="store_true",
                    help="config c3 only: run TimeMix's elementwise parts as torch ops (comparison)")
    ap.add_argument("--serving-modes", default="out_of_place,in_place,graph",
                    help="config c4tm only: which of out_of_place,in_place,graph to run")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (3 launches), to scale rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against known traffic")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": n * 4, "calibrate_copy_bytes_written": n * 4,
                          "launches": 3}))
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(the recurrence shards over batch x heads with no exchange; "
                          "multi-GPU runs are out of scope here)"}))
        sys.exit(2)

    import torch
    from theseus import wkv7 as W
    from theseus.synthetic import wkv7_inputs

    cfg = CONFIGS[args.config]
    if args.config == "c3":
        torch.cuda.set_device(0)
        return bench_timemix(args, cfg)
    if args.config == "c4tm":
        torch.cuda.set_device(0)
        return bench_serving(args, cfg)
    if args.config == "optim":
        torch.cuda.set_device(0)
        return bench_optim(args, cfg)
    if args.config == "gdn":
        torch.cuda.set_device(0)
        return bench_gdn(args, cfg)
    B, T, H, N = cfg["B"], cfg["T"], cfg["H"], cfg["N"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ext = W.extension()
    inp = wkv7_inputs(B, T, H, N, seed=cfg["seed"], dtype=torch.bfloat16, s0_std=cfg["s0_std"])
    xs = [inp[n].to(dev) for n in "rwkvab"]
    s0 = inp["s0"].to(dev)
    dy = inp["dy"].to(dev)
    stream = torch.cuda.current_stream(dev)

    if args.config == "c4":
        # decode: T in-place single steps per "step"; compared with one fused T-step forward
        steps_in = [[x[:, t:t + 1].contiguous() for x in xs] for t in range(T)]
        state = s0.clone()

        def one_step():
            for t in range(T):
                ext.decode_step(*steps_in[t], state)
    elif args.config in ("c2", "n128"):
        def one_step():
            y, end, saved = ext.forward(*xs, s0, True)
            ext.backward(*xs, saved, dy, None)
    else:
        # c1: 8 consecutive T=512 calls with the state carried, no saved states (no-grad path)
        NSPLIT = 8
        Tc = T // NSPLIT
        pieces = [[x[:, i * Tc:(i + 1) * Tc].contiguous() for x in xs] for i in range(NSPLIT)]

        def one_step():
            st = s0
            for pc in pieces:
                _, st, _ = ext.forward(*pc, st, False)
            return st

    def timed(k):
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(k):
            one_step()
        torch.cuda.synchronize()
        return time.perf_counter() - t

    # -- W warmup steps, then K steps timed right after them ------------------------------
    t_warm = time.perf_counter()
    for _ in range(args.warmup):
        one_step()
    ms_after_w = timed(args.steps) * 1e3 / args.steps
    # The MI355X's clocks go through a transient in the first ~20 ms of sustained load
    # (kernel trace of this bench: the same kernels run up to 30 % longer there, with no
    # gap between launches), so the K steps right after W short warmup steps time part of
    # it.  The reported steps come after untimed steps that fill --settle-ms of load.
    extra = max(0, math.ceil((args.settle_ms - (time.perf_counter() - t_warm) * 1e3) / ms_after_w))
    for _ in range(extra):
        one_step()
    settle = args.warmup + args.steps + extra
    torch.cuda.synchronize()

    # -- timed region: exactly K steps ---------------------------------------------------
    elapsed = timed(args.steps)
    ms_per_step = elapsed * 1e3 / args.steps
    tokens = B * T
    value = tokens * args.steps / elapsed

    # -- per-kernel durations with HIP events on the launch stream -----------------------
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    kern = {}
    if args.config == "c4":
        e0, e1 = ev(), ev()
        e0.record(stream)
        for t in range(T):
            ext.decode_step(*steps_in[t], state)
        e1.record(stream)
        torch.cuda.synchronize()
        kern["decode"] = (e0.elapsed_time(e1) / T, alg_bytes(B, 1, H, N, "decode"))
        # the same T tokens as one fused forward (no saved states)
        fused_ms = []
        for _ in range(max(3, min(args.steps, 10))):
            a0, a1 = ev(), ev()
            a0.record(stream)
            ext.forward(*xs, s0, False)
            a1.record(stream)
            torch.cuda.synchronize()
            fused_ms.append(a0.elapsed_time(a1))
        t256_ms = sum(fused_ms) / len(fused_ms)
    elif args.config == "c1":
        # per call: events around each 8-call chain, calls back to back (the launch gaps
        # between a call's kernels included, no host idle time)
        call_ms = []
        for _ in range(max(3, min(args.steps, 10))):
            st = s0
            a0, a1 = ev(), ev()
            a0.record(stream)
            for pc in pieces:
                _, st, _ = ext.forward(*pc, st, False)
            a1.record(stream)
            torch.cuda.synchronize()
            call_ms.append(a0.elapsed_time(a1) / NSPLIT)
        kern["fwd"] = (sum(call_ms) / len(call_ms), alg_bytes(B, Tc, H, N, "fwd"))
        # the same T tokens as one call (no saved states), calls back to back, after an
        # untimed one (its first allocation of the call's outputs and workspace)
        reps = max(3, min(args.steps, 10))
        ext.forward(*xs, s0, False)
        torch.cuda.synchronize()
        a0, a1 = ev(), ev()
        a0.record(stream)
        for _ in range(reps):
            ext.forward(*xs, s0, False)
        a1.record(stream)
        torch.cuda.synchronize()
        single_ms = a0.elapsed_time(a1) / reps
    else:
        fwd_ms, bwd_ms = [], []
        for _ in range(max(3, min(args.steps, 10))):
            a0, a1, a2 = ev(), ev(), ev()
            # keep the stream busy while the host enqueues the timed pair, so that the first
            # interval holds the forward kernel and not the host's launch latency
            if hasattr(torch.cuda, "_sleep"):
                torch.cuda._sleep(1 << 20)
            a0.record(stream)
            y, end, saved = ext.forward(*xs, s0, True)
            a1.record(stream)
            ext.backward(*xs, saved, dy, None)
            a2.record(stream)
            torch.cuda.synchronize()
            fwd_ms.append(a0.elapsed_time(a1))
            bwd_ms.append(a1.elapsed_time(a2))
        kern["fwd"] = (sum(fwd_ms) / len(fwd_ms), alg_bytes(B, T, H, N, "fwd"))
        kern["bwd"] = (sum(bwd_ms) / len(bwd_ms), alg_bytes(B, T, H, N, "bwd"))
    dom = max(kern, key=lambda k: kern[k][0])
    dom_ms, dom_bytes = kern[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9

    if args.config == "c4":
        step_bytes = alg_bytes(B, 1, H, N, "decode") * T
    elif args.config == "c1":
        step_bytes = alg_bytes(B, Tc, H, N, "fwd") * NSPLIT
    else:
        step_bytes = alg_bytes(B, T, H, N, "fwd") + alg_bytes(B, T, H, N, "bwd")
    step_gbps = step_bytes / (ms_per_step * 1e-3) / 1e9

    # HBM bytes per launch, from committed rocprofv3 --pmc runs (FETCH_SIZE and WRITE_SIZE,
    # calibrated against a copy kernel): not measured in this run
    traffic, traffic_src, counted = None, None, None
    tf = ROOT / "profiles" / f"wkv7_{args.config}_traffic.json"
    if tf.exists():
        rec = json.loads(tf.read_text())
        if (rec.get("B"), rec.get("T"), rec.get("H"), rec.get("N")) == (B, T, H, N):
            traffic = rec["bytes_per_launch"].get(dom)
            traffic_src = f"committed rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE: {rec['source']}"
            if all(k in rec["bytes_per_launch"] for k in kern):
                counted = sum(rec["bytes_per_launch"][k] for k in kern)

    cpu = None
    if args.cpu_slice and args.config == "c2":
        cpu = cpu_baseline(B, H, N, args.cpu_slice, cfg["seed"])

    serial_ms = None
    if args.config == "n128":
        # one step on the step-serial kernels (after an untimed one), for comparison
        os.environ["THESEUS_WKV7_FAMILY"] = "seq"
        one_step()
        serial_ms = timed(1) * 1e3
        del os.environ["THESEUS_WKV7_FAMILY"]

    workload = {"c2": "wkv7_fwd_bwd", "n128": "wkv7_fwd_bwd_n128", "c1": "wkv7_fwd_8x512_chained",
                "c4": "wkv7_decode"}[args.config]
    line = {
        "metric": METRIC if args.config == "c2" else f"WKV7 {workload} tokens/s ({args.config})",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "untimed_steps_before_timing": settle,
        "ms_per_step_right_after_warmup": round(ms_after_w, 4),
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "B": B, "T": T, "H": H, "N": N, "io_dtype": "bf16",
                   "state_dtype": "fp32", "checkpoint_interval": ext.checkpoint_interval,
                   "s0_std": cfg["s0_std"], "dsT": "zero", "parallelism": "single-gpu"},
        "hbm_gbps_alg": round(step_gbps, 1),
        "hbm_frac_alg": round(step_gbps / HBM_PEAK_GBPS, 4),
        "kernel_ms": {k: round(v[0], 4) for k, v in kern.items()},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "alg_bytes_per_launch": dom_bytes,
                     "frac_counted": (round(traffic / (dom_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
                                      if traffic else None)},
        "cpu_baseline": cpu,
    }
    if counted:
        # the whole step on counted bytes, and the algorithmic fraction a step could reach at
        # the full 8 TB/s with these bytes (the saved-state traffic the config mandates)
        line["hbm_frac_counted"] = round(counted / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
        line["alg_frac_cap_at_peak"] = round(step_bytes / counted, 4)
    if serial_ms is not None:
        line["step_serial_ms_per_step"] = round(serial_ms, 2)
        line["speedup_vs_step_serial"] = round(serial_ms / ms_per_step, 1)
    if args.config == "c1":
        line["config"].update(calls=NSPLIT, T_per_call=Tc, saved_states=False)
        line["call_ms"] = round(kern["fwd"][0], 4)
        line["single_call_T4096_ms"] = round(single_ms, 4)
    if args.config == "c4":
        line["config"].update(steps_per_call=1, saved_states=False)
        line["decode_step_ms"] = round(kern["decode"][0], 4)
        line["fused_t256_forward_ms"] = round(t256_ms, 4)
        line["decode_over_fused_t256"] = round(kern["decode"][0] * T / t256_ms, 2)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
