"""Weight-format producers and reference dequantisers (torch, any device).

Same API and semantics as src/paia_gemv/quant.py:8-38 (the reference's formats, defined in quant_host.h):
  FP8 W8A16  e4m3fn weights, one fp32 scale per output row: scale = amax/448 (1 if the row is all zero),
             q = e4m3_rn(clamp(W/scale, +-448)).
  INT4 W4A16 unsigned nibbles, zero point 8, group 128 along K, fp16 scale = fp16(amax/7) (1 if zero);
             n = clamp(rint(w/s), -7, 7) + 8 with s = float(scale) (1 where the fp16 scale underflowed to 0);
             byte j of a row = weight 2j (low nibble) | weight 2j+1 (high nibble).
The quantizers run the library's HIP kernels for a tensor on the GPU (paia_gemv.ops.quantize_*, bit-identical to
these definitions; they raise if the extension is missing) and the torch definitions below for a CPU tensor. The
dequantisers are the torch definitions on either device (paia_gemv.ops.dequant_* runs them as HIP kernels).

Additions for the asymmetric INT4 format of the BASELINE configurations (no reference counterpart):
  `quantize_int4_zp_g128(W)` per group of 128: lo = min(0, min w), hi = max(0, max w), s = bf16((hi - lo) / 15)
                            (1 if that is 0), z = clamp(rint(-lo / s), 0, 15), q = clamp(rint(w / s) + z, 0, 15)
  `pack_int4(q)`            q uint8 [N,K] in 0..15 -> packed uint8 [N,K/2] (same nibble order as above)
  `pack_zeros(z)`           z uint8 [N,G] in 0..15 -> uint8 [N,ceil(G/2)], group 2j low nibble, 2j+1 high
  `dequant_int4_zp(p, s, z)` (q - z) * float(s_bf16), fp32 [N,K]
"""
import torch


def quantize_fp8_rowwise(W):
    """W [N,K] float32 -> (q uint8 [N,K], scale float32 [N])."""
    if W.is_cuda:
        from . import ops
        return ops.quantize_fp8_rowwise(W.float().contiguous())
    amax = W.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)).float()
    q = (W / scale[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), scale


def dequant_fp8(q, scale):
    """float(e4m3(q)) * scale[n] -> fp32 [N,K]."""
    return q.view(torch.float8_e4m3fn).float() * scale[:, None]


def quantize_int4_g128(W):
    """W [N,K] float32, K % 128 == 0 -> (packed uint8 [N,K/2], scales float16 [N,K/128])."""
    N, K = W.shape
    if K % 128:
        raise ValueError("K % 128 required")
    if W.is_cuda:
        from . import ops
        return ops.quantize_int4_g128(W.float().contiguous())
    grp = W.reshape(N, K // 128, 128)
    amax = grp.abs().amax(dim=-1)
    s16 = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax)).to(torch.float16)
    sf = s16.float()
    sf = torch.where(sf > 0, sf, torch.ones_like(sf))
    n = (torch.round(grp / sf[..., None]).clamp(-7, 7) + 8).to(torch.uint8).reshape(N, K)
    return pack_int4(n), s16.contiguous()


def dequant_int4(packed, s16):
    """(n - 8) * float(s16) -> fp32 [N,K]."""
    n = unpack_int4(packed).float()
    return (n - 8.0) * s16.float().repeat_interleave(128, dim=1)


def quantize_int4_zp_g128(W):
    """W [N,K] float32, K % 128 == 0 -> (packed uint8 [N,K/2], scales bf16 [N,G], zeros uint8 [N,ceil(G/2)]),
    dequantising as (q - z) * s."""
    N, K = W.shape
    if K % 128:
        raise ValueError("K % 128 required")
    if W.is_cuda:
        from . import ops
        return ops.quantize_int4_zp_g128(W.float().contiguous())
    grp = W.float().reshape(N, K // 128, 128)
    lo = grp.amin(dim=-1).clamp(max=0.0)
    hi = grp.amax(dim=-1).clamp(min=0.0)
    sb = ((hi - lo) / 15.0).to(torch.bfloat16)
    sb = torch.where(sb.float() > 0, sb, torch.ones_like(sb))
    s = sb.float()
    z = torch.round(-lo / s).clamp(0, 15)
    q = (torch.round(grp / s[..., None]) + z[..., None]).clamp(0, 15).to(torch.uint8).reshape(N, K)
    return pack_int4(q), sb.contiguous(), pack_zeros(z.to(torch.uint8))


def pack_int4(q):
    """q uint8 [N,K] with values 0..15, K even -> [N,K/2]: byte j = q[2j] | q[2j+1] << 4 (8 per int32 along K)."""
    q = q.to(torch.uint8)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()


def unpack_int4(packed):
    """[N,K/2] -> uint8 [N,K] nibbles (inverse of pack_int4)."""
    N, half = packed.shape
    p = packed.to(torch.uint8)
    return torch.stack([p & 0xF, p >> 4], dim=-1).reshape(N, 2 * half)


def pack_zeros(z):
    """z uint8 [N,G] with values 0..15 -> [N,ceil(G/2)]: byte j = z[2j] | z[2j+1] << 4 (odd G: high nibble 0)."""
    N, G = z.shape
    z = z.to(torch.uint8)
    if G % 2:
        z = torch.cat([z, torch.zeros(N, 1, dtype=torch.uint8, device=z.device)], dim=1)
    return (z[:, 0::2] | (z[:, 1::2] << 4)).contiguous()


def unpack_zeros(zp, G):
    N = zp.shape[0]
    p = zp.to(torch.uint8)
    return torch.stack([p & 0xF, p >> 4], dim=-1).reshape(N, -1)[:, :G]


def dequant_int4_zp(packed, scales_bf16, zeros):
    """(q - z) * float(s_bf16) -> fp32 [N,K]; scales bf16 [N,G], zeros packed [N,ceil(G/2)]."""
    q = unpack_int4(packed).float()
    G = scales_bf16.shape[1]
    z = unpack_zeros(zeros, G).float().repeat_interleave(128, dim=1)
    return (q - z) * scales_bf16.float().repeat_interleave(128, dim=1)
