// A GEMM on preloaded operands: X [256 x 512] and W [512 x 384] arrive in a preload image (the reference's HBM
// preload format, softhier_mlir_amd/preload.py), the sentinel segment last; run as `preload_gemm.exe --preload <image>`.
builtin.module {
  func.func @preload_gemm() {
    %x = softhier.hbm_buffer {offset = 4096 : i32} : memref<256x512xf16, "hbm_west">
    %w = softhier.hbm_buffer {offset = 266240 : i32} : memref<512x384xf16, "hbm_west">
    %z = softhier.hbm_buffer {offset = 659456 : i32} : memref<256x384xf16, "hbm_west">
    %s = softhier.hbm_buffer {offset = 856064 : i32} : memref<1x32xf16, "hbm_west">
    softhier.preload_wait %s : memref<1x32xf16, "hbm_west">
    softhier.gemm %x, %w into %z {fmt = "fp16", tile_m = 256 : i32, tile_n = 128 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32}
        : memref<256x512xf16, "hbm_west">, memref<512x384xf16, "hbm_west">, memref<256x384xf16, "hbm_west">
    softhier.dump_samples %z {seed = 41 : i32, n = 128 : i32, tag = "Z"} : memref<256x384xf16, "hbm_west">
    func.return
  }
}
