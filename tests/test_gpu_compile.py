"""The ops behave as torch custom ops must for the way the reference runs them: torch.library.opcheck on
every op (schema, fake kernels, AOT dispatch with dynamic shapes), and torch.compile(fullgraph=True, mode="max-autotune") of a decoder-layer stack of
BF16RotateLinearWrapper / SharedInputRotateLinears modules, replayed as CUDA graphs the way the reference
drives its compiled language model (alpamayo_r1_unified.py:404-409, 486-493; fake kernels as in
kernels/paroquant_kernels/__init__.py:7-27)."""

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.paroquant_kernels import scaled_pairwise_rotation
from alpamayo_amd.quantization import SharedInputRotateLinears
from tests.gpu_util import packed_rotation

pytestmark = pytest.mark.gpu


def _operands(N, K, seed):
    g = workloads.generator(seed)
    spec = workloads.linear_spec("x", N, K, g)
    rot_idx, rot_cs, _, _ = packed_rotation(spec.pairs, spec.theta)
    wp, wm = torch.ops.paroquant.w4a8_prepack(spec.w.awq_qweight.cuda(), spec.w.awq_scales.cuda(),
                                              spec.w.awq_qzeros.cuda())
    s, sz = workloads.w16_scales(spec.w)
    wp16, wm16 = torch.ops.paroquant.w4a16_prepack(spec.w.awq_qweight.cuda(), s.cuda(), sz.cuda())
    return dict(spec=spec, rot_idx=rot_idx.cuda(), rot_cs=rot_cs.cuda(),
                sc=spec.channel_scales.float().reshape(-1).cuda(), wp=wp, wm=wm, wp16=wp16, wm16=wm16)


def _opcheck_cases():
    K, bf = 256, torch.bfloat16
    a = _operands(64, K, 8100)
    b = _operands(48, K, 8101)
    sp = a["spec"]
    x = workloads.activations(5, K, workloads.generator(8102)).cuda()
    x16 = x.half()
    idx, th, cs = sp.pairs.cuda(), sp.theta.to(bf).cuda(), sp.channel_scales.to(bf).cuda()
    xq, xs = torch.ops.paroquant.rotate_quant_i8(x, a["rot_idx"], a["rot_cs"], a["sc"], 8, True, True)
    grp = lambda key: [a[key], b[key]]   # noqa: E731
    w = sp.w
    return {
        "rotate": (torch.ops.rotation.rotate, (x, idx, th, cs, 128)),
        "rotate_and_quant_mxfp4": (torch.ops.rotation.rotate_and_quant_mxfp4, (x, idx, th, cs, 128)),
        "rotate_backward": (torch.ops.paroquant.rotate_backward, (x.clone(), x, idx, th, cs, 128)),
        "rotate_quant_i8": (torch.ops.paroquant.rotate_quant_i8, (x, a["rot_idx"], a["rot_cs"], a["sc"], 8, True,
                                                                  True)),
        "rotate_quant_i8_rot": (torch.ops.paroquant.rotate_quant_i8_rot, (x, a["rot_idx"], a["rot_cs"], None, 8,
                                                                          False, True)),
        "quant_i8": (torch.ops.paroquant.quant_i8, (x,)),
        "w4a8_prepack": (torch.ops.paroquant.w4a8_prepack, (w.awq_qweight.cuda(), w.awq_scales.cuda(),
                                                            w.awq_qzeros.cuda())),
        "w4a8_gemm": (torch.ops.paroquant.w4a8_gemm, (xq, xs, a["wp"], a["wm"], None, bf)),
        "w4a8_gemm_partials": (torch.ops.paroquant.w4a8_gemm_partials, (xq, a["wp"], a["wm"])),
        "w4a8_linear": (torch.ops.paroquant.w4a8_linear, (x, a["rot_idx"], a["rot_cs"], a["sc"], 8, a["wp"], a["wm"],
                                                          None, True, True, bf)),
        "w4a8_linear_group": (torch.ops.paroquant.w4a8_linear_group,
                              (x, grp("rot_idx"), grp("rot_cs"), grp("sc"), 8, grp("wp"), grp("wm"), [None, None],
                               True, True, bf)),
        "w4a8_linear_group_rmsnorm": (torch.ops.paroquant.w4a8_linear_group_rmsnorm,
                                      (x, x.clone(), torch.ones(K, dtype=bf, device="cuda"), 1e-6, grp("rot_idx"),
                                       grp("rot_cs"), grp("sc"), 8, grp("wp"), grp("wm"), [None, None], True,
                                       True, bf, True, True)),
        "w4a8_linear_group_fused": (torch.ops.paroquant.w4a8_linear_group_fused,
                                    (x, x.clone(), None, 0.0, 3, grp("rot_idx"), grp("rot_cs"), grp("sc"), 8,
                                     grp("wp"), grp("wm"), [None, None], True, True, bf, True, False)),
        "w4a16_prepack": (torch.ops.paroquant.w4a16_prepack,
                          (w.awq_qweight.cuda(), *(t.cuda() for t in workloads.w16_scales(w)))),
        "w4a16_gemm": (torch.ops.paroquant.w4a16_gemm, (x16, a["wp16"], a["wm16"], None, torch.float16)),
        "w4a16_linear": (torch.ops.paroquant.w4a16_linear, (x16, a["rot_idx"], a["rot_cs"], a["sc"], 8, a["wp16"],
                                                            a["wm16"], None, False, torch.float16)),
        "w4a16_linear_group": (torch.ops.paroquant.w4a16_linear_group,
                               (x, grp("rot_idx"), grp("rot_cs"), grp("sc"), 8, grp("wp16"), grp("wm16"),
                                [None, None], True, bf)),
    }


def test_opcheck_every_op():
    cases = _opcheck_cases()
    registered = {n.split("::")[1].split(".")[0] for n in torch._C._dispatch_get_all_op_names()
                  if n.startswith(("paroquant::", "rotation::"))}
    assert {"rotate", "w4a8_linear", "rotate_backward"} <= registered
    assert registered <= set(cases), f"ops without an opcheck case: {registered - set(cases)}"
    for name, (op, args) in cases.items():
        print(f"opcheck {name}", flush=True)
        torch.library.opcheck(op, args)


def _decoder_stack(n_layers, dev):
    """n_layers Qwen3-8B decoder layers' quantized linears as the benchmark's verify block chains them."""
    class Layer(torch.nn.Module):
        def __init__(self, seed):
            super().__init__()
            g = workloads.generator(seed, device=dev)
            mods = [workloads.build_module(workloads.linear_spec(n, N, K, g, device=dev), dev)
                    for n, (N, K) in workloads.QWEN3_8B_LINEARS.items()]
            self.qkv = SharedInputRotateLinears(mods[0:3])
            self.o = mods[3]
            self.gu = SharedInputRotateLinears(mods[4:6])
            self.down = SharedInputRotateLinears(mods[6:7])
            self.register_buffer("w_norm", (0.8 + 0.4 * torch.rand(4096, generator=g, device=dev)).to(torch.bfloat16))

    class Stack(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = torch.nn.ModuleList([Layer(8200 + i) for i in range(n_layers)])

        def forward(self, a):
            h = d = None
            for L in self.layers:
                if d is None:
                    q, k, v = L.qkv(a)
                else:
                    q, k, v, a = L.qkv(h, residual=d, return_sum=True)
                o = L.o(q)
                gt, up, h = L.gu(o, norm_weight=L.w_norm, eps=1e-6, residual=a, return_normed=True)
                (d,) = L.down.forward_swiglu(gt, up)
            return h + d

    return Stack()


def _eager_like_inductor(stack, a):
    """The stack's forward in eager mode, with silu(gate) * up on the prefill path formed in float32 and
    rounded once, as inductor fuses it (eager torch rounds silu's result first).  Every kernel of this
    package is the same in both; only that torch-side step differs.  The difference is one bf16 ulp on
    about a quarter of the products, which random int4 layers amplify to a few percent of the output."""
    from alpamayo_amd import ops

    h = d = None
    for L in stack.layers:
        if d is None:
            q, k, v = L.qkv(a)
        else:
            q, k, v, a = L.qkv(h, residual=d, return_sum=True)
        o = L.o(q)
        gt, up, h = L.gu(o, norm_weight=L.w_norm, eps=1e-6, residual=a, return_normed=True)
        if ops.split_path(gt.numel() // gt.size(-1), gt.size(-1)):
            (d,) = L.down.forward_swiglu(gt, up)
        else:
            (d,) = L.down(((torch.nn.functional.silu(gt.float()) * up.float()).to(gt.dtype)))
    return h + d


@pytest.mark.timeout(900)
def test_compiled_decoder_stack_replays_match_eager():
    dev = torch.device("cuda")
    stack = _decoder_stack(2, dev)
    compiled = torch.compile(stack, fullgraph=True, mode="max-autotune")
    for M in (16, 1, 96):
        print(f"compiled stack M={M}", flush=True)
        a = workloads.activations(M, 4096, workloads.generator(8300 + M, device=dev), device=dev)
        eager = _eager_like_inductor(stack, a)
        outs = []
        for _ in range(3):
            torch.compiler.cudagraph_mark_step_begin()
            outs.append(compiled(a).clone())
            stack(a + 1)          # eager work between the replays
        torch.cuda.synchronize()
        for y in outs:
            assert torch.equal(y, eager), f"M={M}: compiled replay differs from eager"


def test_compiled_wrapper_and_rotation_backward():
    dev = torch.device("cuda")
    spec = workloads.linear_spec("v_proj", 1024, 4096, workloads.generator(8400))
    mod = workloads.build_module(spec, dev)
    x = workloads.activations(8, 4096, workloads.generator(8401)).cuda()
    eager = mod(x)
    cm = torch.compile(mod, fullgraph=True)
    assert torch.equal(cm(x), eager)

    rng = np.random.default_rng(5)
    pairs = torch.from_numpy(np.stack([np.concatenate([rng.permutation(128) for _ in range(4)]) for _ in range(8)])
                             .astype(np.int16)).cuda()
    theta = torch.from_numpy(rng.uniform(-3, 3, (8, 256)).astype(np.float32)).cuda()
    scales = torch.from_numpy(rng.uniform(0.5, 2, (1, 512)).astype(np.float32)).cuda()
    xr = torch.from_numpy(rng.standard_normal((33, 512)).astype(np.float32)).cuda()
    w = torch.from_numpy(rng.standard_normal((33, 512)).astype(np.float32)).cuda()

    def loss(x_, t_, s_):
        return (scaled_pairwise_rotation(x_, pairs, t_, s_, 128) * w).sum()

    grads = []
    for fn in (loss, torch.compile(loss, fullgraph=True)):
        leaves = [t.clone().requires_grad_(True) for t in (xr, theta, scales)]
        fn(*leaves).backward()
        grads.append([t.grad for t in leaves])
    for ge, gc in zip(*grads):
        assert torch.equal(ge, gc)
