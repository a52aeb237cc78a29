"""Seeded synthetic inputs for the measured configurations.

Every generator draws from ``numpy.random.default_rng(seed)`` in a fixed order, so a seed
names one exact input.  The configuration seeds are ``SEED_BASE + config_index`` with the
configurations numbered 1..5 as listed in the benchmark definition:

1. Q6_K GEMV 5120x5120, fp32 x (M=1)
2. IQ3_XXS FFN gate+up + SwiGLU, K=5120, N=2x17408, M in {1,4,8,11}
3. dense decode-step weight sweep at M=11 (64 layers + Q6_K head)
4. prefill IQ3_XXS FFN dequant-GEMM at M in {2048, 8192}
5. MoE grouped IQ4_XS (256 experts + 1 shared, top-8) at M in {11, 2048}

Block field rules (all bytes not listed are uniform): ``d = fp16(|N(0,1)| * 1e-3)``;
Q6_K ``sc`` uniform int8; IQ3_XXS grid-index bytes uniform over 0..255 and scale/sign
words uniform over 32 bits; IQ4_XS scale and index bytes uniform.
"""
import numpy as np

SEED_BASE = 20261201


def config_rng(config_index):
    return np.random.default_rng(SEED_BASE + config_index)


def _d16(rng, shape):
    return (np.abs(rng.standard_normal(shape)) * 1e-3).astype(np.float16)


def q6k_raw(rng, rows, kdim):
    """GGUF Q6_K rows u8[rows, 210*NB]: ql/qh bytes, then sc, then d."""
    nb = kdim // 256
    qlqh = rng.integers(0, 256, size=(rows, nb, 192), dtype=np.uint8)
    sc = rng.integers(-128, 128, size=(rows, nb, 16)).astype(np.int8)
    d = _d16(rng, (rows, nb))
    blk = np.empty((rows, nb, 210), dtype=np.uint8)
    blk[:, :, 0:192] = qlqh
    blk[:, :, 192:208] = sc.view(np.uint8)
    blk[:, :, 208:210] = d.view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 210)


def k4_raw(rng, rows, kdim, five):
    """GGUF Q4_K (five=False, 144*NB B) or Q5_K (176*NB B) rows: d and dmin as above, then
    uniform scale, qh and qs bytes."""
    nb = kdim // 256
    nbytes = 176 if five else 144
    d = _d16(rng, (rows, nb, 2))
    rest = rng.integers(0, 256, size=(rows, nb, nbytes - 4), dtype=np.uint8)
    blk = np.empty((rows, nb, nbytes), dtype=np.uint8)
    blk[:, :, 0:4] = d.view(np.uint8).reshape(rows, nb, 4)
    blk[:, :, 4:] = rest
    return blk.reshape(rows, nb * nbytes)


def iq3xxs_raw(rng, rows, kdim):
    """GGUF IQ3_XXS rows u8[rows, 98*NB]: d, then grid-index bytes, then scale/sign words."""
    nb = kdim // 256
    d = _d16(rng, (rows, nb))
    qs = rng.integers(0, 256, size=(rows, nb, 64), dtype=np.uint8)
    sw = rng.integers(0, 1 << 32, size=(rows, nb, 8), dtype=np.uint64).astype("<u4")
    blk = np.empty((rows, nb, 98), dtype=np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:66] = qs
    blk[:, :, 66:98] = sw.view(np.uint8).reshape(rows, nb, 32)
    return blk.reshape(rows, nb * 98)


def iq4xs_raw(rng, rows, kdim):
    """GGUF IQ4_XS rows u8[rows, 136*NB]: d, then scales_h/scales_l/qs bytes."""
    nb = kdim // 256
    d = _d16(rng, (rows, nb))
    rest = rng.integers(0, 256, size=(rows, nb, 134), dtype=np.uint8)
    blk = np.empty((rows, nb, 136), dtype=np.uint8)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:136] = rest
    return blk.reshape(rows, nb * 136)


def bf16_round(x):
    """float32 -> the nearest bfloat16 value (round half to even), returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> 16) & 1)) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def activations_f16(rng, m, k):
    """bf16 N(0,1) activations quantized to fp16 the way the reference feeds its kernels
    (round-to-nearest-even ``__float2half``)."""
    return bf16_round(rng.standard_normal((m, k)).astype(np.float32)).astype(np.float16)


def moe_expert_slabs(rng, n_experts):
    """Config 5 expert weights: per expert a gate/up slab u8[2*512*1088] (512 gate rows, then
    512 up rows, k = 2048) and a down slab u8[2048*272] (k = 512), GGUF IQ4_XS rows."""
    gu = [np.concatenate([iq4xs_raw(rng, 512, 2048).ravel(), iq4xs_raw(rng, 512, 2048).ravel()])
          for _ in range(n_experts)]
    dn = [iq4xs_raw(rng, 2048, 512).ravel() for _ in range(n_experts)]
    return gu, dn


def iq3s_raw(rng, rows, kdim):
    """GGUF IQ3_S rows u8[rows, 110*NB]: d, then index / high-bit / sign / scale bytes uniform."""
    nb = kdim // 256
    blk = rng.integers(0, 256, size=(rows, nb, 110), dtype=np.uint8)
    blk[:, :, 0:2] = _d16(rng, (rows, nb)).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 110)


def iq3s_grid(rng):
    """A synthetic IQ3_S grid float32[512, 4] with ggml's level set (odd 1..15).  The real table
    is a third-party constant absent here; the kernels take the grid at run time."""
    return rng.choice(np.arange(1, 16, 2), size=(512, 4)).astype(np.float32)


def q80_raw(rng, rows, kdim):
    """GGUF Q8_0 rows u8[rows, 34*(kdim/32)]: d, then 32 int8 uniform."""
    nb = kdim // 32
    blk = np.empty((rows, nb, 34), dtype=np.uint8)
    blk[:, :, 2:34] = rng.integers(0, 256, size=(rows, nb, 32), dtype=np.uint8)
    blk[:, :, 0:2] = _d16(rng, (rows, nb)).view(np.uint8).reshape(rows, nb, 2)
    return blk.reshape(rows, nb * 34)


def moe_ckpt_slabs(rng, n_experts):
    """The checkpoint's MoE classes: per routed expert an IQ3_S gate/up slab u8[2*512*880] (512
    gate rows, then 512 up rows, k = 2048) and a Q6_K down slab u8[2048*420] (k = 512); the shared
    expert's Q8_0 gate, up (512 x 2176 B) and down (2048 x 544 B) rows."""
    gu = [np.concatenate([iq3s_raw(rng, 512, 2048).ravel(), iq3s_raw(rng, 512, 2048).ravel()])
          for _ in range(n_experts)]
    dn = [q6k_raw(rng, 2048, 512).ravel() for _ in range(n_experts)]
    shared = (q80_raw(rng, 512, 2048), q80_raw(rng, 512, 2048), q80_raw(rng, 2048, 512))
    return gu, dn, shared
