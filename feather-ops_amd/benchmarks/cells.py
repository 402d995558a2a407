"""The shape grid the scaled_mm tile heuristic is fitted on.

A cell is `(M, N, K)`: M activation rows against a weight of N outputs over K inputs (the GEMM is
[M, K] x [K, N]). The grid is the reference's benchmark grid (`bench/cells.py:30-96` in the reference:
real (out, in) pairs of the diffusion and text models its consumers run, at their activation-row bands,
plus a resolution ladder and the weight-streaming cells), so a tile rule fitted here is fitted on the
same workload, plus the five benchmark configurations of this build as the `baseline` group.
"""

# 16x-VAE token counts for 512^2 ... 2048^2 images, plus 16 packed text rows.
_M_512, _M_768, _M_1024, _M_1280, _M_1536, _M_2048 = 1040, 2320, 4112, 6416, 9232, 16400

GROUPS: dict[str, list[tuple[int, int, int]]] = {
    # The benchmark configurations (C1..C5) of this build.
    "baseline": [(256, 1024, 1024), (4096, 3072, 3072), (4096, 12288, 3072), (16, 14336, 4096),
                 (1, 1000, 2560), (77, 5120, 2560), (1000, 1000, 2560), (4097, 5120, 2560)],
    # Resolution ladder on three weight classes.
    "ladder-wide": [(m, 6144, 6144) for m in (_M_512, _M_768, _M_1280, _M_2048)] + [(_M_1024, 6144, 6144),
                                                                                   (_M_1536, 6144, 6144)],
    "ladder-narrow": [(m, 1536, 6144) for m in (_M_512, _M_768, _M_1024, _M_1280, _M_1536, _M_2048)],
    "ladder-small": [(m, 1024, 5120) for m in (_M_512, _M_768, _M_1024, _M_1536, _M_2048)],
    "sdxl": [(1024, 1280, 1280), (1024, 10240, 1280), (2304, 1280, 1280), (2304, 10240, 1280),
             (4096, 1280, 5120), (9216, 1280, 5120), (4096, 5120, 1280)],
    "anima": [(512, 1024, 1024), (512, 2048, 1024), (4096, 2048, 2048), (4096, 8192, 2048),
              (4096, 2048, 8192), (9216, 2048, 2048), (9216, 8192, 2048), (4096, 1024, 4096)],
    "qwen21": [(4096, 3072, 12288), (9216, 18432, 3072)],
    "qwen2_1": [(2, 4096, 16384), (16, 4096, 4096), (4112, 4096, 4096), (4112, 4096, 12288),
                (4112, 24576, 4096), (9232, 16384, 4096), (9232, 4096, 4096)],
    "zimage": [(32, 3840, 2560), (4128, 3840, 3840), (4128, 11520, 3840), (4128, 3840, 10240),
               (9248, 10240, 3840), (9248, 3840, 3840)],
    "krea2": [(16, 6144, 6144), (192, 1536, 6144), (4112, 6144, 16384), (4112, 16384, 6144),
              (4112, 2560, 6912)],
    "ideogram4": [(4096, 4608, 4608), (4096, 4608, 12288), (4096, 4608, 53248), (9232, 12288, 4608),
                  (9232, 18432, 512)],
    "klein9b": [(512, 4096, 4096), (4096, 4096, 4096), (4096, 4096, 12288), (4608, 36864, 4096),
                (4608, 4096, 16384), (9216, 12288, 4096), (9728, 4096, 4096)],
    "wan": [(512, 5120, 5120), (512, 13824, 5120), (12032, 5120, 5120), (12032, 5120, 13824),
            (12032, 30720, 5120)],
    "ltx2_3": [(1024, 4096, 4096), (1536, 4096, 4096), (8960, 4096, 16384), (8960, 8192, 4096)],
    "h3": [(16, 5376, 5376), (512, 5376, 5120), (5251, 21504, 5376), (5376, 21504, 5376),
           (5376, 5376, 7168), (5376, 28672, 5376), (5376, 5376, 14336), (25343, 21504, 5376),
           (25344, 21504, 5376)],
    "moss": [(4112, 9216, 3072), (4112, 3072, 3072), (4112, 16384, 3072), (9232, 3072, 8192),
             (9232, 18432, 3072)],
    "short-prompt": [(32, 25600, 5120), (32, 5120, 25600), (128, 1024, 5120), (128, 8192, 5120)],
    "text-16": [(16, 3072, 3072)],
    "pad-256": [(192, 2560, 2560), (256, 2560, 2560), (192, 12288, 4096), (256, 12288, 4096),
                (256, 4096, 4096)],
    "text-1152": [(512, 1152, 1152), (2048, 1152, 1152), (2048, 1152, 4304), (2048, 4304, 1152),
                  (4096, 3456, 1152)],
    "weight-stream": [(512, 248320, 4096), (1, 96768, 2688)],
}


def cells(groups: set[str] | None = None) -> list[tuple[str, int, int, int]]:
    """`[(group, M, N, K)]` for the whole grid or the named groups; a cell belongs to one group only."""
    selected = [(name, m, n, k) for name, shapes in GROUPS.items() if groups is None or name in groups
                for m, n, k in shapes]
    shapes = [(m, n, k) for _, m, n, k in selected]
    if len(set(shapes)) != len(shapes):
        repeated = sorted({s for s in shapes if shapes.count(s) > 1})
        raise ValueError(f"the grid repeats cells: {repeated}")
    return selected
