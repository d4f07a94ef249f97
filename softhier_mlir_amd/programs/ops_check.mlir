// Row ops, a GEMM on strided head views and a fused attention on views of a QKV buffer, with LCG test inputs
// and sampled outputs ("<tag> r c hex" lines) that tests/test_gpu_programs.py compares with the oracle.
builtin.module {
  func.func @ops_check() {
    %x = softhier.hbm_buffer {offset = 0 : i32} : memref<256x768xf16, "hbm_west">
    %g = softhier.hbm_buffer {offset = 393216 : i32} : memref<1x768xf16, "hbm_west">
    %be = softhier.hbm_buffer {offset = 397312 : i32} : memref<1x768xf16, "hbm_west">
    %y = softhier.hbm_buffer {offset = 401408 : i32} : memref<256x768xf16, "hbm_west">
    %kT = softhier.hbm_buffer {offset = 794624 : i32} : memref<768x256xf16, "hbm_west">
    %s = softhier.hbm_buffer {offset = 1187840 : i32} : memref<256x256xf16, "hbm_west">
    %ge = softhier.hbm_buffer {offset = 1318912 : i32} : memref<256x768xf16, "hbm_west">
    %ab = softhier.hbm_buffer {offset = 1712128 : i32} : memref<256x768xf16, "hbm_west">
    %ad = softhier.hbm_buffer {offset = 2105344 : i32} : memref<256x768xf16, "hbm_west">
    %qkv = softhier.hbm_buffer {offset = 2498560 : i32} : memref<256x2304xf16, "hbm_west">
    %o = softhier.hbm_buffer {offset = 3678208 : i32} : memref<256x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %x {seed = 1 : i32, lo = -16 : i32, hi = 16 : i32, scale = 0.125 : f32} : memref<256x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %g {seed = 14 : i32, lo = 2 : i32, hi = 6 : i32, scale = 0.25 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %be {seed = 15 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.125 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %qkv {seed = 21 : i32, lo = -16 : i32, hi = 16 : i32, scale = 0.0625 : f32} : memref<256x2304xf16, "hbm_west">
    softhier.layernorm %x, %g, %be -> %y {eps = 1.0e-6 : f32, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
    softhier.transpose %y -> %kT {cluster = -1 : i32} : memref<256x768xf16, "hbm_west"> -> memref<768x256xf16, "hbm_west">
    %q1 = softhier.view %y : memref<256x768xf16, "hbm_west"> -> memref<256x64xf16, strided<[768, 1], offset: 64>, "hbm_west">
    %k1 = softhier.view %kT : memref<768x256xf16, "hbm_west"> -> memref<64x256xf16, strided<[256, 1], offset: 16384>, "hbm_west">
    softhier.gemm %q1, %k1 into %s {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 64 : i32, pipeline, cluster = 1 : i32} : memref<256x64xf16, strided<[768, 1], offset: 64>, "hbm_west">, memref<64x256xf16, strided<[256, 1], offset: 16384>, "hbm_west">, memref<256x256xf16, "hbm_west">
    softhier.softmax %s -> %s {scale = 0.125 : f32, cluster = 1 : i32} : memref<256x256xf16, "hbm_west"> -> memref<256x256xf16, "hbm_west">
    softhier.gelu %y -> %ge {cluster = -1 : i32} : memref<256x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
    softhier.add_bias %ge, %be -> %ab {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
    softhier.add %x, %ab -> %ad {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
    %q = softhier.view %qkv : memref<256x2304xf16, "hbm_west"> -> memref<256x768xf16, strided<[2304, 1], offset: 0>, "hbm_west">
    %k = softhier.view %qkv : memref<256x2304xf16, "hbm_west"> -> memref<256x768xf16, strided<[2304, 1], offset: 768>, "hbm_west">
    %v = softhier.view %qkv : memref<256x2304xf16, "hbm_west"> -> memref<256x768xf16, strided<[2304, 1], offset: 1536>, "hbm_west">
    softhier.attention %q, %k, %v -> %o {scale = 0.125 : f32, heads = 12 : i32, cluster = -1 : i32} : memref<256x768xf16, strided<[2304, 1], offset: 0>, "hbm_west">, memref<256x768xf16, strided<[2304, 1], offset: 768>, "hbm_west">, memref<256x768xf16, strided<[2304, 1], offset: 1536>, "hbm_west"> -> memref<256x768xf16, "hbm_west">
    softhier.dump_samples %y {seed = 31 : i32, n = 96 : i32, tag = "Y"} : memref<256x768xf16, "hbm_west">
    softhier.dump_samples %kT {seed = 32 : i32, n = 96 : i32, tag = "KT"} : memref<768x256xf16, "hbm_west">
    softhier.dump_samples %s {seed = 33 : i32, n = 96 : i32, tag = "S"} : memref<256x256xf16, "hbm_west">
    softhier.dump_samples %ge {seed = 34 : i32, n = 96 : i32, tag = "GE"} : memref<256x768xf16, "hbm_west">
    softhier.dump_samples %ab {seed = 35 : i32, n = 96 : i32, tag = "AB"} : memref<256x768xf16, "hbm_west">
    softhier.dump_samples %ad {seed = 36 : i32, n = 96 : i32, tag = "AD"} : memref<256x768xf16, "hbm_west">
    softhier.dump_samples %o {seed = 37 : i32, n = 96 : i32, tag = "O"} : memref<256x768xf16, "hbm_west">
    func.return
  }
}
