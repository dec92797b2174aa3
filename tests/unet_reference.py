"""float32 CPU reference of the SD-UNet workloads (mtorch_amd.sd_unet) for the parity tests.

torch-CPU float32 stands in as the "fp32 CPU" reference the C4/C5 parity bar names: the block
and UNet compositions are this repository's SD-1.5 workloads (the reference ships no UNet), and
every op in them is one whose device kernel is separately pinned against the oracle.  Weights
are read from the device model, widened exactly to float32."""

import numpy as np
import torch
import torch.nn.functional as TF

import mtorch_amd as mt
from mtorch_amd import sd_unet


class Weights:
    def __init__(self):
        self.cache = {}

    def __call__(self, p):
        if p is None:
            return None
        key = id(p)
        if key not in self.cache:
            a = p.cpu().float().numpy() if p.dtype is mt.float16 else p.cpu().numpy()
            self.cache[key] = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
        return self.cache[key]


def t32(x):
    """Device tensor -> torch float32 (exact widening)."""
    a = x.cpu().float().numpy() if x.dtype is mt.float16 else x.cpu().numpy()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def resblock(W, blk, x, temb_silu):
    h = TF.conv2d(TF.silu(TF.group_norm(x, 32, W(blk.norm1.weight), W(blk.norm1.bias), blk.norm1.eps)),
                  W(blk.conv1.weight), W(blk.conv1.bias), padding=1)
    h = h + TF.linear(temb_silu, W(blk.time_emb_proj.weight), W(blk.time_emb_proj.bias))[:, :, None, None]
    h = TF.conv2d(TF.silu(TF.group_norm(h, 32, W(blk.norm2.weight), W(blk.norm2.bias), blk.norm2.eps)),
                  W(blk.conv2.weight), W(blk.conv2.bias), padding=1)
    res = TF.conv2d(x, W(blk.shortcut.weight), W(blk.shortcut.bias)) if blk.shortcut is not None else x
    return res + h


def attention(W, att, h, context=None):
    B, L, C = h.shape
    heads = att.heads
    if att.self_attn:
        qkv = TF.linear(h, W(att.to_qkv.weight))
        q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
    else:
        q = TF.linear(h, W(att.to_q.weight))
        kv = TF.linear(context, W(att.to_kv.weight))
        k, v = kv[..., :C], kv[..., C:]

    def split(t):
        return t.reshape(B, t.shape[1], heads, C // heads).transpose(1, 2).contiguous()

    o = TF.scaled_dot_product_attention(split(q), split(k), split(v))
    o = o.transpose(1, 2).reshape(B, L, C)
    return TF.linear(o, W(att.to_out.weight), W(att.to_out.bias))


def transformer(W, blk, x, context):
    B, C, H, Wd = x.shape
    h = TF.group_norm(x, 32, W(blk.norm.weight), W(blk.norm.bias), blk.norm.eps)
    h = TF.conv2d(h, W(blk.proj_in.weight), W(blk.proj_in.bias))
    tok = h.reshape(B, C, H * Wd).transpose(1, 2)
    tok = tok + attention(W, blk.attn1, TF.layer_norm(tok, [C], W(blk.norm1.weight), W(blk.norm1.bias)))
    tok = tok + attention(W, blk.attn2, TF.layer_norm(tok, [C], W(blk.norm2.weight), W(blk.norm2.bias)), context)
    ff = TF.linear(TF.layer_norm(tok, [C], W(blk.norm3.weight), W(blk.norm3.bias)), W(blk.ff_in.weight),
                   W(blk.ff_in.bias))
    a, gate = ff.chunk(2, dim=-1)
    tok = tok + TF.linear(a * TF.gelu(gate), W(blk.ff_out.weight), W(blk.ff_out.bias))
    h = tok.transpose(1, 2).reshape(B, C, H, Wd)
    return TF.conv2d(h, W(blk.proj_out.weight), W(blk.proj_out.bias)) + x


def unet(W, model, latent, t, context):
    freqs = t32(model.freqs)
    args = t.reshape(-1, 1) * freqs.reshape(1, -1)
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    emb = TF.linear(TF.silu(TF.linear(emb, W(model.time1.weight), W(model.time1.bias))), W(model.time2.weight),
                    W(model.time2.bias))
    temb_silu = TF.silu(emb)
    h = TF.conv2d(latent, W(model.conv_in.weight), W(model.conv_in.bias), padding=1)
    skips = [h]

    def run(items, h, with_skip):
        i = 0
        while i < len(items):
            blk = items[i]
            if isinstance(blk, sd_unet.ResBlock):
                x = torch.cat([h, skips.pop()], dim=1) if not with_skip else h
                h = resblock(W, blk, x, temb_silu)
                if i + 1 < len(items) and isinstance(items[i + 1], sd_unet.SpatialTransformer):
                    i += 1
                    h = transformer(W, items[i], h, context)
            elif isinstance(blk, sd_unet.Downsample):
                h = TF.conv2d(h, W(blk.conv.weight), W(blk.conv.bias), stride=2, padding=1)
            else:
                h = TF.conv2d(TF.interpolate(h, scale_factor=2, mode="nearest"), W(blk.conv.weight), W(blk.conv.bias),
                              padding=1)
            if with_skip:
                skips.append(h)
            i += 1
        return h

    for blocks in model.down:
        h = run(list(blocks), h, True)
    h = resblock(W, model.mid[0], h, temb_silu)
    h = transformer(W, model.mid[1], h, context)
    h = resblock(W, model.mid[2], h, temb_silu)
    for blocks in model.up:
        h = run(list(blocks), h, False)
    n = model.norm_out
    h = TF.silu(TF.group_norm(h, 32, W(n.weight), W(n.bias), n.eps))
    return TF.conv2d(h, W(model.conv_out.weight), W(model.conv_out.bias), padding=1)


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))
