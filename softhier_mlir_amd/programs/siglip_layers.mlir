// Two SigLIP-B encoder layers (S = 256, D = 768, 12 heads, FFN 3072) in the reference's op order, as a loop over
// layer-indexed weight buffers (layer L's parameters at offset + L * stride, LCG-filled with the reference's seed
// table: layer L adds 100 L). The residual stream %x is updated in place; each layer dumps samples of it.
builtin.module {
  func.func @siglip_layers() {
    %c0 = arith.constant 0 : index
    %c1 = arith.constant 1 : index
    %cL = arith.constant 2 : index
    %x = softhier.hbm_buffer {offset = 0 : i32} : memref<256x768xf16, "hbm_west">
    %ln1 = softhier.hbm_buffer {offset = 393216 : i32} : memref<256x768xf16, "hbm_west">
    %q = softhier.hbm_buffer {offset = 786432 : i32} : memref<256x768xf16, "hbm_west">
    %k = softhier.hbm_buffer {offset = 1179648 : i32} : memref<256x768xf16, "hbm_west">
    %v = softhier.hbm_buffer {offset = 1572864 : i32} : memref<256x768xf16, "hbm_west">
    %o = softhier.hbm_buffer {offset = 1966080 : i32} : memref<256x768xf16, "hbm_west">
    %ao = softhier.hbm_buffer {offset = 2359296 : i32} : memref<256x768xf16, "hbm_west">
    %h = softhier.hbm_buffer {offset = 2752512 : i32} : memref<256x768xf16, "hbm_west">
    %ln2 = softhier.hbm_buffer {offset = 3145728 : i32} : memref<256x768xf16, "hbm_west">
    %f1 = softhier.hbm_buffer {offset = 3538944 : i32} : memref<256x3072xf16, "hbm_west">
    %g = softhier.hbm_buffer {offset = 5111808 : i32} : memref<256x3072xf16, "hbm_west">
    %f2 = softhier.hbm_buffer {offset = 6684672 : i32} : memref<256x768xf16, "hbm_west">
    %wq_0 = softhier.hbm_buffer {offset = 7077888 : i32} : memref<768x768xf16, "hbm_west">
    %wk_0 = softhier.hbm_buffer {offset = 8257536 : i32} : memref<768x768xf16, "hbm_west">
    %wv_0 = softhier.hbm_buffer {offset = 9437184 : i32} : memref<768x768xf16, "hbm_west">
    %wo_0 = softhier.hbm_buffer {offset = 10616832 : i32} : memref<768x768xf16, "hbm_west">
    %w1_0 = softhier.hbm_buffer {offset = 11796480 : i32} : memref<768x3072xf16, "hbm_west">
    %w2_0 = softhier.hbm_buffer {offset = 16515072 : i32} : memref<3072x768xf16, "hbm_west">
    %bq_0 = softhier.hbm_buffer {offset = 21233664 : i32} : memref<1x768xf16, "hbm_west">
    %bk_0 = softhier.hbm_buffer {offset = 21237760 : i32} : memref<1x768xf16, "hbm_west">
    %bv_0 = softhier.hbm_buffer {offset = 21241856 : i32} : memref<1x768xf16, "hbm_west">
    %bo_0 = softhier.hbm_buffer {offset = 21245952 : i32} : memref<1x768xf16, "hbm_west">
    %b1_0 = softhier.hbm_buffer {offset = 21250048 : i32} : memref<1x3072xf16, "hbm_west">
    %b2_0 = softhier.hbm_buffer {offset = 21258240 : i32} : memref<1x768xf16, "hbm_west">
    %g1_0 = softhier.hbm_buffer {offset = 21262336 : i32} : memref<1x768xf16, "hbm_west">
    %be1_0 = softhier.hbm_buffer {offset = 21266432 : i32} : memref<1x768xf16, "hbm_west">
    %g2_0 = softhier.hbm_buffer {offset = 21270528 : i32} : memref<1x768xf16, "hbm_west">
    %be2_0 = softhier.hbm_buffer {offset = 21274624 : i32} : memref<1x768xf16, "hbm_west">
    %wq_1 = softhier.hbm_buffer {offset = 21278720 : i32} : memref<768x768xf16, "hbm_west">
    %wk_1 = softhier.hbm_buffer {offset = 22458368 : i32} : memref<768x768xf16, "hbm_west">
    %wv_1 = softhier.hbm_buffer {offset = 23638016 : i32} : memref<768x768xf16, "hbm_west">
    %wo_1 = softhier.hbm_buffer {offset = 24817664 : i32} : memref<768x768xf16, "hbm_west">
    %w1_1 = softhier.hbm_buffer {offset = 25997312 : i32} : memref<768x3072xf16, "hbm_west">
    %w2_1 = softhier.hbm_buffer {offset = 30715904 : i32} : memref<3072x768xf16, "hbm_west">
    %bq_1 = softhier.hbm_buffer {offset = 35434496 : i32} : memref<1x768xf16, "hbm_west">
    %bk_1 = softhier.hbm_buffer {offset = 35438592 : i32} : memref<1x768xf16, "hbm_west">
    %bv_1 = softhier.hbm_buffer {offset = 35442688 : i32} : memref<1x768xf16, "hbm_west">
    %bo_1 = softhier.hbm_buffer {offset = 35446784 : i32} : memref<1x768xf16, "hbm_west">
    %b1_1 = softhier.hbm_buffer {offset = 35450880 : i32} : memref<1x3072xf16, "hbm_west">
    %b2_1 = softhier.hbm_buffer {offset = 35459072 : i32} : memref<1x768xf16, "hbm_west">
    %g1_1 = softhier.hbm_buffer {offset = 35463168 : i32} : memref<1x768xf16, "hbm_west">
    %be1_1 = softhier.hbm_buffer {offset = 35467264 : i32} : memref<1x768xf16, "hbm_west">
    %g2_1 = softhier.hbm_buffer {offset = 35471360 : i32} : memref<1x768xf16, "hbm_west">
    %be2_1 = softhier.hbm_buffer {offset = 35475456 : i32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %x {seed = 1 : i32, lo = -16 : i32, hi = 16 : i32, scale = 0.125 : f32} : memref<256x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wq_0 {seed = 2 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wk_0 {seed = 3 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wv_0 {seed = 4 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wo_0 {seed = 5 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %w1_0 {seed = 6 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x3072xf16, "hbm_west">
    softhier.hbm_fill_lcg %w2_0 {seed = 7 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.00390625 : f32} : memref<3072x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bq_0 {seed = 8 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bk_0 {seed = 9 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bv_0 {seed = 10 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bo_0 {seed = 11 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %b1_0 {seed = 12 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x3072xf16, "hbm_west">
    softhier.hbm_fill_lcg %b2_0 {seed = 13 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %g1_0 {seed = 14 : i32, lo = 2 : i32, hi = 6 : i32, scale = 0.25 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %be1_0 {seed = 15 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.125 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %g2_0 {seed = 16 : i32, lo = 2 : i32, hi = 6 : i32, scale = 0.25 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %be2_0 {seed = 17 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.125 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wq_1 {seed = 102 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wk_1 {seed = 103 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wv_1 {seed = 104 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %wo_1 {seed = 105 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %w1_1 {seed = 106 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.0078125 : f32} : memref<768x3072xf16, "hbm_west">
    softhier.hbm_fill_lcg %w2_1 {seed = 107 : i32, lo = -8 : i32, hi = 8 : i32, scale = 0.00390625 : f32} : memref<3072x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bq_1 {seed = 108 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bk_1 {seed = 109 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bv_1 {seed = 110 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %bo_1 {seed = 111 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %b1_1 {seed = 112 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x3072xf16, "hbm_west">
    softhier.hbm_fill_lcg %b2_1 {seed = 113 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.0625 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %g1_1 {seed = 114 : i32, lo = 2 : i32, hi = 6 : i32, scale = 0.25 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %be1_1 {seed = 115 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.125 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %g2_1 {seed = 116 : i32, lo = 2 : i32, hi = 6 : i32, scale = 0.25 : f32} : memref<1x768xf16, "hbm_west">
    softhier.hbm_fill_lcg %be2_1 {seed = 117 : i32, lo = -4 : i32, hi = 4 : i32, scale = 0.125 : f32} : memref<1x768xf16, "hbm_west">
    scf.for %L = %c0 to %cL step %c1 {
      %L1 = arith.addi %L, %c1 : index
      %wq = softhier.hbm_buffer %L {offset = 7077888 : i32, stride = 14200832 : i32} : memref<768x768xf16, "hbm_west">
      %wk = softhier.hbm_buffer %L {offset = 8257536 : i32, stride = 14200832 : i32} : memref<768x768xf16, "hbm_west">
      %wv = softhier.hbm_buffer %L {offset = 9437184 : i32, stride = 14200832 : i32} : memref<768x768xf16, "hbm_west">
      %wo = softhier.hbm_buffer %L {offset = 10616832 : i32, stride = 14200832 : i32} : memref<768x768xf16, "hbm_west">
      %w1 = softhier.hbm_buffer %L {offset = 11796480 : i32, stride = 14200832 : i32} : memref<768x3072xf16, "hbm_west">
      %w2 = softhier.hbm_buffer %L {offset = 16515072 : i32, stride = 14200832 : i32} : memref<3072x768xf16, "hbm_west">
      %bq = softhier.hbm_buffer %L {offset = 21233664 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %bk = softhier.hbm_buffer %L {offset = 21237760 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %bv = softhier.hbm_buffer %L {offset = 21241856 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %bo = softhier.hbm_buffer %L {offset = 21245952 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %b1 = softhier.hbm_buffer %L {offset = 21250048 : i32, stride = 14200832 : i32} : memref<1x3072xf16, "hbm_west">
      %b2 = softhier.hbm_buffer %L {offset = 21258240 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %g1 = softhier.hbm_buffer %L {offset = 21262336 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %be1 = softhier.hbm_buffer %L {offset = 21266432 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %g2 = softhier.hbm_buffer %L {offset = 21270528 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      %be2 = softhier.hbm_buffer %L {offset = 21274624 : i32, stride = 14200832 : i32} : memref<1x768xf16, "hbm_west">
      softhier.layernorm %x, %g1, %be1 -> %ln1 {eps = 1.0e-6 : f32, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.gemm %ln1, %wq into %q {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<768x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">
      softhier.add_bias %q, %bq -> %q {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.gemm %ln1, %wk into %k {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<768x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">
      softhier.add_bias %k, %bk -> %k {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.gemm %ln1, %wv into %v {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<768x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">
      softhier.add_bias %v, %bv -> %v {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.attention %q, %k, %v -> %o {scale = 0.125 : f32, heads = 12 : i32, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.gemm %o, %wo into %ao {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<768x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">
      softhier.add_bias %ao, %bo -> %ao {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.add %x, %ao -> %h {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.layernorm %h, %g2, %be2 -> %ln2 {eps = 1.0e-6 : f32, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.gemm %ln2, %w1 into %f1 {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<768x3072xf16, "hbm_west">, memref<256x3072xf16, "hbm_west">
      softhier.add_bias %f1, %b1 -> %f1 {cluster = -1 : i32} : memref<256x3072xf16, "hbm_west">, memref<1x3072xf16, "hbm_west"> -> memref<256x3072xf16, "hbm_west">
      softhier.gelu %f1 -> %g {cluster = -1 : i32} : memref<256x3072xf16, "hbm_west"> -> memref<256x3072xf16, "hbm_west">
      softhier.gemm %g, %w2 into %f2 {fmt = "fp16", tile_m = 256 : i32, tile_n = 256 : i32, tile_k = 256 : i32, pipeline, cluster = -1 : i32} : memref<256x3072xf16, "hbm_west">, memref<3072x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west">
      softhier.add_bias %f2, %b2 -> %f2 {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<1x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.add %h, %f2 -> %x {cluster = -1 : i32} : memref<256x768xf16, "hbm_west">, memref<256x768xf16, "hbm_west"> -> memref<256x768xf16, "hbm_west">
      softhier.mark %L1 {tag = "layer"}
      softhier.dump_samples %x, %L1 {seed = 205 : i32, n = 128 : i32, tag = "OUT"} : memref<256x768xf16, "hbm_west">
    }
    func.return
  }
}
