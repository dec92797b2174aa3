"""SD-1.5-shaped UNet workloads on the device: the SpatialTransformer block (BASELINE.json
configs[3]) and the full conditional UNet, written against this package's operator
surface the way an mtorch user would write them, using its fused device paths where an SD
pipeline's op sequence allows (GroupNorm+SiLU+conv, linear+residual, GEGLU).

Architecture (Stable Diffusion 1.5): channels (320, 640, 1280, 1280), two ResNet blocks per
level, a SpatialTransformer (8 heads, cross-attention on a [B, 77, 768] context) after each
ResNet block of the first three levels and in the middle block, nearest x2 upsampling, 3x3
stride-2 downsampling, sinusoidal 320-d timestep embedding -> Linear(320, 1280) -> SiLU ->
Linear(1280, 1280).  ~860 M parameters.

Dtypes follow the usual fp16 SD deployment: weights and activations fp16, the norm layers' own
parameters fp32 with the upcast pattern norm(x.float(), w32, b32).half().

Layout: activations stay NCHW between blocks (the reference's observable layout).  Inside a
ResNet block the GroupNorm+SiLU output goes channels-last straight into the conv; inside a
transformer block the channels-last GroupNorm output *is* the [B, HW, C] token tensor, the
attention writes its heads merged back into tokens, and proj_out reads the tokens as an NHWC
1x1 conv whose epilogue adds the NCHW residual.
"""

from __future__ import annotations

import math

import numpy as np

from . import _lib
from . import _ops
from . import _tensor as T
from . import nn
from ._tensor import Tensor

F = nn.functional


# ------------------------------------------------------------------------------ parameters


class _Init:
    """Random N(0, std) initialisation from mtorch's generator, drawn per parameter in the
    parameter's own dtype (fp16 draws round each value once, as the reference's fp16 normal_
    does) and uploaded to the device."""

    def __init__(self, device: str, std: float = 0.02):
        self.device = device
        self.std = std

    def normal(self, *shape, dtype=T.float16) -> nn.Parameter:
        t = T.empty(*shape, dtype=dtype)
        t.normal_(0.0, self.std)
        return nn.Parameter(t.to(self.device), requires_grad=False)

    def const(self, value: float, *shape, dtype=T.float32) -> nn.Parameter:
        return nn.Parameter(T.full(list(shape), value, dtype=dtype).to(self.device), requires_grad=False)


class _GN(nn.Module):
    def __init__(self, init: _Init, C: int, eps: float):
        super().__init__()
        self.weight = init.const(1.0, C)
        self.bias = init.const(0.0, C)
        self.groups = 32
        self.eps = eps


class _Conv(nn.Module):
    def __init__(self, init: _Init, cin: int, cout: int, k: int):
        super().__init__()
        self.weight = init.normal(cout, cin, k, k)
        self.bias = init.normal(cout)


class _Linear(nn.Module):
    def __init__(self, init: _Init, cin: int, cout: int, bias: bool = True):
        super().__init__()
        self.weight = init.normal(cout, cin)
        self.bias = init.normal(cout) if bias else None


# ------------------------------------------------------------------------------ blocks


def _tokens_nhwc(x: Tensor, norm: _GN) -> Tensor:
    """group_norm(x.float(), ...).half() written channels-last: the [B, H*W, C] token tensor
    that permute(0, 2, 3, 1).reshape(B, H*W, C) of the NCHW result would give."""
    B, C, H, W = x.shape
    dev = x._dev()
    out = _ops._empty([B, H * W, C], x.dtype, dev)
    if C % (8 if x.dtype is T.float16 else 4):
        raise ValueError("token layout needs the channel count to be a multiple of 8")
    pdt = _ops._norm_param_dtype("group_norm", x, norm.weight, norm.bias)
    _lib.check(_lib.lib().mthip_group_norm_nhwc(dev, x.dtype.code, x.contiguous().data_ptr(), norm.weight.data_ptr(),
                                                norm.bias.data_ptr(), out.data_ptr(), B, C, H * W, norm.groups,
                                                float(norm.eps), 0, pdt))
    return out


def _attention_tokens(q: Tensor, k: Tensor, v: Tensor, heads: int) -> Tensor:
    """Multi-head attention on token tensors: q[B, Lq, C], k/v[B, Lk, C] (any row stride, unit
    channel stride; e.g. column slices of a fused QKV projection), heads of C/heads channels.
    Returns [B, Lq, C] -- sdpa(q.view(B,Lq,h,d).transpose(1,2), ...).transpose(1,2).reshape(B,Lq,C)
    with the heads merged by the kernel's output strides instead of a copy."""
    B, Lq, C = q.shape
    Lk = k.shape[1]
    D = C // heads
    dev = q._dev()
    out = _ops._empty([B, Lq, C], q.dtype, dev)
    for t in (q, k, v):
        if t.stride(2) != 1:
            raise ValueError("token tensors need a unit channel stride")
    a = _lib.int64_array
    _lib.check(_lib.lib().mthip_sdpa(dev, q.dtype.code, q.data_ptr(), a([q.stride(0), D, q.stride(1)]), k.data_ptr(),
                                     a([k.stride(0), D, k.stride(1)]), v.data_ptr(), a([v.stride(0), D, v.stride(1)]),
                                     out.data_ptr(), a([Lq * C, D, C]), B, heads, heads, Lq, Lk, D, D, 0,
                                     _lib.F32, None, None, 0, 0, 0.0))
    return out


def _layer_norm(x: Tensor, norm: nn.Module) -> Tensor:
    return _ops.layer_norm(x, [x.shape[-1]], norm.weight, norm.bias, 1e-5, allow_upcast=True)


class _LN(nn.Module):
    def __init__(self, init: _Init, C: int):
        super().__init__()
        self.weight = init.const(1.0, C)
        self.bias = init.const(0.0, C)


class ResBlock(nn.Module):
    """GN -> SiLU -> conv3x3 (+ time embedding) -> GN -> SiLU -> conv3x3 (+ shortcut)."""

    def __init__(self, init: _Init, cin: int, cout: int, temb: int = 1280):
        super().__init__()
        self.norm1 = _GN(init, cin, 1e-5)
        self.conv1 = _Conv(init, cin, cout, 3)
        self.time_emb_proj = _Linear(init, temb, cout)
        self.norm2 = _GN(init, cout, 1e-5)
        self.conv2 = _Conv(init, cout, cout, 3)
        self.shortcut = _Conv(init, cin, cout, 1) if cin != cout else None

    def forward(self, x: Tensor, temb_silu: Tensor, t: Tensor | None = None) -> Tensor:
        """t: this block's time projection linear(temb_silu) when the caller computed it already
        (the UNet runs every block's projection as one GEMM)."""
        n1, n2 = self.norm1, self.norm2
        if t is None:
            t = F.linear(temb_silu, self.time_emb_proj.weight, self.time_emb_proj.bias)
        r = None
        if self.shortcut is not None:
            # the GroupNorm also writes x channels-last for the shortcut conv
            r = _ops.group_norm_silu_conv2d_cat(x, None, n1.groups, n1.weight, n1.bias, n1.eps, self.conv1.weight,
                                                self.conv1.bias, 1, t, self.shortcut.weight, self.shortcut.bias)
        if r is not None:
            h, res = r
        else:
            # h = conv1(silu(norm1(x))) + t[:, :, None, None], the add in conv1's epilogue
            h = F.group_norm_silu_conv2d(x, n1.groups, n1.weight, n1.bias, n1.eps, self.conv1.weight,
                                         self.conv1.bias, padding=1, chan_add=t)
            res = F.conv2d(x, self.shortcut.weight, self.shortcut.bias) if self.shortcut is not None else x
        return F.group_norm_silu_conv2d(h, n2.groups, n2.weight, n2.bias, n2.eps, self.conv2.weight, self.conv2.bias,
                                        padding=1, residual=res)

    def forward_cat(self, x0: Tensor, x1: Tensor, temb_silu: Tensor, t: Tensor | None = None) -> Tensor:
        """forward(cat([x0, x1], dim=1), ...) of an up-block ResBlock without the concatenated
        copy: the first GroupNorm reads both inputs in place and also hands the shortcut conv its
        channels-last operand."""
        n1, n2 = self.norm1, self.norm2
        if t is None:
            t = F.linear(temb_silu, self.time_emb_proj.weight, self.time_emb_proj.bias)
        r = None
        if self.shortcut is not None:
            r = _ops.group_norm_silu_conv2d_cat(x0, x1, n1.groups, n1.weight, n1.bias, n1.eps, self.conv1.weight,
                                                self.conv1.bias, 1, t, self.shortcut.weight, self.shortcut.bias)
        if r is None:
            return self.forward(_ops.cat([x0, x1], dim=1), temb_silu, t)
        h, res = r
        return F.group_norm_silu_conv2d(h, n2.groups, n2.weight, n2.bias, n2.eps, self.conv2.weight, self.conv2.bias,
                                        padding=1, residual=res)


class Attention(nn.Module):
    def __init__(self, init: _Init, C: int, ctx: int | None, heads: int = 8):
        super().__init__()
        self.heads = heads
        self.self_attn = ctx is None
        if self.self_attn:
            self.to_qkv = _Linear(init, C, 3 * C, bias=False)  # to_q, to_k, to_v stacked
        else:
            self.to_q = _Linear(init, C, C, bias=False)
            self.to_kv = _Linear(init, ctx, 2 * C, bias=False)  # to_k, to_v stacked
        self.to_out = _Linear(init, C, C)

    def forward(self, h: Tensor, residual: Tensor, context: Tensor | None = None, kv: Tensor | None = None) -> Tensor:
        """kv: this block's context projection linear(context, to_kv) when the caller computed
        it already (the UNet projects the context for every cross-attention in one GEMM)."""
        C = h.shape[-1]
        if self.self_attn:
            qkv = F.linear(h, self.to_qkv.weight)
            q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
        else:
            q = F.linear(h, self.to_q.weight)
            if kv is None:
                kv = F.linear(context, self.to_kv.weight)
            k, v = kv[..., :C], kv[..., C:]
        o = _attention_tokens(q, k, v, self.heads)
        return F.linear_residual(o, self.to_out.weight, self.to_out.bias, residual)


class SpatialTransformer(nn.Module):
    """GN -> proj_in (1x1) -> [LN -> self-attn, LN -> cross-attn, LN -> GEGLU FFN] -> proj_out
    (1x1) + residual."""

    def __init__(self, init: _Init, C: int, ctx: int = 768, heads: int = 8):
        super().__init__()
        self.norm = _GN(init, C, 1e-6)
        self.proj_in = _Conv(init, C, C, 1)
        self.norm1 = _LN(init, C)
        self.attn1 = Attention(init, C, None, heads)
        self.norm2 = _LN(init, C)
        self.attn2 = Attention(init, C, ctx, heads)
        self.norm3 = _LN(init, C)
        self.ff_in = _Linear(init, C, 8 * C)
        self.ff_out = _Linear(init, 4 * C, C)
        self.proj_out = _Conv(init, C, C, 1)

    def forward(self, x: Tensor, context: Tensor, kv: Tensor | None = None) -> Tensor:
        B, C, H, W = x.shape
        tok = _tokens_nhwc(x, self.norm)
        tok = F.linear(tok, self.proj_in.weight.view(C, C), self.proj_in.bias)
        tok = self.attn1(_layer_norm(tok, self.norm1), tok)
        tok = self.attn2(_layer_norm(tok, self.norm2), tok, context, kv)
        ff = F.linear_geglu(_layer_norm(tok, self.norm3), self.ff_in.weight, self.ff_in.bias)
        tok = F.linear_residual(ff, self.ff_out.weight, self.ff_out.bias, tok)
        return _ops.conv2d_tokens(tok, self.proj_out.weight, self.proj_out.bias, H, W, residual=x)


class Downsample(nn.Module):
    def __init__(self, init: _Init, C: int):
        super().__init__()
        self.conv = _Conv(init, C, C, 3)

    def forward(self, x):
        return F.conv2d(x, self.conv.weight, self.conv.bias, stride=2, padding=1)


class Upsample(nn.Module):
    def __init__(self, init: _Init, C: int):
        super().__init__()
        self.conv = _Conv(init, C, C, 3)

    def forward(self, x):
        y = _ops.upsample2x_conv2d(x, self.conv.weight, self.conv.bias, padding=1)
        if y is not None:
            return y
        return F.conv2d(F.interpolate(x, scale_factor=2, mode="nearest"), self.conv.weight, self.conv.bias, padding=1)


def timestep_frequencies(dim: int = 320, device: str = "cuda") -> Tensor:
    """f = exp(-log(10000) * arange(dim/2) / (dim/2)), evaluated in fp32 in the reference's op
    order (tests/compat/benchmarking.py:6014-6019) once on the host, then kept on the device."""
    half = dim // 2
    exponent = -np.log(np.float32(10000.0)) * np.arange(half, dtype=np.float32) / np.float32(half)
    return T.from_numpy(np.exp(exponent).astype(np.float32)).to(device)


def timestep_embedding(t: Tensor, freqs: Tensor) -> Tensor:
    """[cos(t f), sin(t f)] in fp32 (tests/compat/benchmarking.py:6031-6032); device ops only,
    so a captured step can take the timestep as a device tensor."""
    import mtorch_amd as mt

    args = t.reshape(-1, 1) * freqs.reshape(1, -1)
    return mt.cat([args.cos(), args.sin()], dim=-1)


def timestep_embedding_f16(t: Tensor, freqs: Tensor) -> Tensor:
    """timestep_embedding(t, freqs).half() in one launch (mthip_timestep_embedding_f16, the same
    values bit for bit) for fp32 timesteps and frequencies on the device; otherwise the op
    sequence."""
    if t.dtype is T.float32 and freqs.dtype is T.float32 and t.dim() == 1 and freqs.dim() == 1 and t.is_cuda:
        dev = _ops._gpu("timestep_embedding", t, freqs)
        B, half = t.shape[0], freqs.shape[0]
        out = _ops._empty([B, 2 * half], T.float16, dev)
        _lib.check(_lib.lib().mthip_timestep_embedding_f16(dev, t.contiguous().data_ptr(), freqs.contiguous().data_ptr(),
                                                           out.data_ptr(), B, half))
        return out
    return timestep_embedding(t, freqs).half()


class UNet(nn.Module):
    """Stable-Diffusion-1.5-shaped conditional UNet, fp16, random N(0, 0.02) weights."""

    def __init__(self, seed: int = 0, device: str = "cuda", ch=(320, 640, 1280, 1280), ctx: int = 768):
        super().__init__()
        import mtorch_amd as mt

        mt.manual_seed(seed)
        init = _Init(device)
        self.conv_in = _Conv(init, 4, ch[0], 3)
        self.time1 = _Linear(init, ch[0], 4 * ch[0])
        self.time2 = _Linear(init, 4 * ch[0], 4 * ch[0])
        temb = 4 * ch[0]
        self.down = nn.ModuleList()
        skips = [ch[0]]
        cin = ch[0]
        for level, c in enumerate(ch):
            blocks = nn.ModuleList()
            for _ in range(2):
                blocks.append(ResBlock(init, cin, c, temb))
                if level < 3:
                    blocks.append(SpatialTransformer(init, c, ctx))
                cin = c
                skips.append(c)
            if level < 3:
                blocks.append(Downsample(init, c))
                skips.append(c)
            self.down.append(blocks)
        self.mid = nn.ModuleList([ResBlock(init, ch[3], ch[3], temb), SpatialTransformer(init, ch[3], ctx),
                                  ResBlock(init, ch[3], ch[3], temb)])
        self.up = nn.ModuleList()
        rev = list(reversed(ch))
        for level, c in enumerate(rev):
            blocks = nn.ModuleList()
            for _ in range(3):
                blocks.append(ResBlock(init, cin + skips.pop(), c, temb))
                if level > 0:
                    blocks.append(SpatialTransformer(init, c, ctx))
                cin = c
            if level < 3:
                blocks.append(Upsample(init, c))
            self.up.append(blocks)
        self.norm_out = _GN(init, ch[0], 1e-5)
        self.conv_out = _Conv(init, ch[0], 4, 3)
        self.freqs = timestep_frequencies(ch[0], device)
        object.__setattr__(self, "_stack_cache", {})

    def _stacked(self, name: str, linears) -> tuple:
        """Weights (and biases) of several linears that read the same input, concatenated along
        the output dimension so they run as one GEMM; rebuilt whenever one of the parameters
        was written in place (storage version), like the packed conv weights."""
        import mtorch_amd as mt

        params = [p for lin in linears for p in (lin.weight, lin.bias) if p is not None]
        key = tuple((id(p._storage), p._storage.version) for p in params)
        hit = self._stack_cache.get(name)
        if hit is None or hit[0] != key:
            w = mt.cat([lin.weight for lin in linears], dim=0)
            b = mt.cat([lin.bias for lin in linears], dim=0) if linears[0].bias is not None else None
            offs = np.cumsum([0] + [lin.weight.shape[0] for lin in linears]).tolist()
            hit = (key, w, b, offs)
            self._stack_cache[name] = hit
        return hit[1], hit[2], hit[3]

    def _blocks(self):
        for blocks in list(self.down) + [self.mid] + list(self.up):
            yield from blocks

    def forward(self, latent: Tensor, timesteps: Tensor, context: Tensor) -> Tensor:
        import mtorch_amd as mt

        emb = timestep_embedding_f16(timesteps, self.freqs)
        emb = F.linear_silu(emb, self.time1.weight, self.time1.bias)
        # every ResBlock's time projection reads silu(emb), and nothing reads emb itself: the
        # SiLU rides in the second linear's epilogue
        temb_silu = F.linear_silu(emb, self.time2.weight, self.time2.bias)
        # all ResBlock time projections as one GEMM, all cross-attention K/V projections as another
        res_blocks = [b for b in self._blocks() if isinstance(b, ResBlock)]
        tw, tb, toff = self._stacked("time", [b.time_emb_proj for b in res_blocks])
        t_all = F.linear(temb_silu, tw, tb)
        t_of = {id(b): t_all[:, toff[i]:toff[i + 1]] for i, b in enumerate(res_blocks)}
        xf_blocks = [b for b in self._blocks() if isinstance(b, SpatialTransformer)]
        kw, _, koff = self._stacked("kv", [b.attn2.to_kv for b in xf_blocks])
        kv_all = F.linear(context, kw)
        kv_of = {id(b): kv_all[..., koff[i]:koff[i + 1]] for i, b in enumerate(xf_blocks)}

        def res(blk, x):
            return blk(x, temb_silu, t_of[id(blk)])

        def xf(blk, x):
            return blk(x, context, kv_of[id(blk)])

        h = F.conv2d(latent, self.conv_in.weight, self.conv_in.bias, padding=1)
        skips = [h]
        for blocks in self.down:
            items = list(blocks)
            i = 0
            while i < len(items):
                if isinstance(items[i], ResBlock):
                    h = res(items[i], h)
                    if i + 1 < len(items) and isinstance(items[i + 1], SpatialTransformer):
                        i += 1
                        h = xf(items[i], h)
                else:  # Downsample
                    h = items[i](h)
                skips.append(h)
                i += 1
        h = res(self.mid[0], h)
        h = xf(self.mid[1], h)
        h = res(self.mid[2], h)
        for blocks in self.up:
            items = list(blocks)
            i = 0
            while i < len(items):
                if isinstance(items[i], ResBlock):
                    blk = items[i]
                    h = blk.forward_cat(h, skips.pop(), temb_silu, t_of[id(blk)])
                    if i + 1 < len(items) and isinstance(items[i + 1], SpatialTransformer):
                        i += 1
                        h = xf(items[i], h)
                else:  # Upsample
                    h = items[i](h)
                i += 1
        n = self.norm_out
        return F.group_norm_silu_conv2d(h, n.groups, n.weight, n.bias, n.eps, self.conv_out.weight, self.conv_out.bias,
                                        padding=1)


def unet_flops(ch=(320, 640, 1280, 1280), B: int = 2, HW: int = 64, ctx_len: int = 77, ctx: int = 768,
               parts: dict | None = None) -> float:
    """Algorithmic FLOP of one UNet forward (2 per MAC; convs, linears and attention products).
    parts (optional) receives the split by op family: "conv3x3", "conv1x1" (proj_in/out and
    the ResBlock shortcuts), "linear" (projections, feed-forward, time MLPs) and "attention"
    (the QK^T and PV products)."""
    acc = {"conv3x3": 0.0, "conv1x1": 0.0, "linear": 0.0, "attention": 0.0}

    def conv(cin, cout, k, hw):
        f = 2.0 * B * hw * hw * cout * cin * k * k
        acc["conv3x3" if k == 3 else "conv1x1"] += f

    def linear(f):
        acc["linear"] += f

    def transformer(C, hw):
        L = hw * hw
        conv(C, C, 1, hw)  # proj_in
        conv(C, C, 1, hw)  # proj_out
        linear(2.0 * B * L * C * 3 * C + 2.0 * B * L * C * C)  # qkv, out (self)
        acc["attention"] += 4.0 * B * L * L * C  # self attention QK^T and PV
        linear(2.0 * B * L * C * C + 2.0 * B * ctx_len * ctx * 2 * C + 2.0 * B * L * C * C)  # q, kv, out (cross)
        acc["attention"] += 4.0 * B * L * ctx_len * C
        linear(2.0 * B * L * C * 8 * C + 2.0 * B * L * 4 * C * C)  # GEGLU in, FF out

    def res(cin, cout, hw):
        conv(cin, cout, 3, hw)
        conv(cout, cout, 3, hw)
        linear(2.0 * B * 4 * ch[0] * cout)  # time embedding projection
        if cin != cout:
            conv(cin, cout, 1, hw)

    conv(4, ch[0], 3, HW)
    linear(2.0 * B * (ch[0] * 4 * ch[0] + 4 * ch[0] * 4 * ch[0]))
    hw, cin, skips = HW, ch[0], [ch[0]]
    for level, c in enumerate(ch):
        for _ in range(2):
            res(cin, c, hw)
            if level < 3:
                transformer(c, hw)
            cin = c
            skips.append(c)
        if level < 3:
            conv(c, c, 3, hw // 2)
            hw //= 2
            skips.append(c)
    res(ch[3], ch[3], hw)
    res(ch[3], ch[3], hw)
    transformer(ch[3], hw)
    for level, c in enumerate(reversed(ch)):
        for _ in range(3):
            res(cin + skips.pop(), c, hw)
            if level > 0:
                transformer(c, hw)
            cin = c
        if level < 3:
            hw *= 2
            conv(c, c, 3, hw)
    conv(ch[0], 4, 3, HW)
    if parts is not None:
        parts.update(acc)
    return sum(acc.values())
