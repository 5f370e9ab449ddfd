/* A host program with no Python and no torch that drives the HIP path through
 * the C ABI alone, as a cgo / JNI / N-API binding would: device buffers from
 * hipMalloc, inputs from raw little-endian files, one call per entry point,
 * outputs back to raw files. tests/test_gpu_c_host.py writes the inputs and
 * checks the outputs.
 *
 *   tc_host decode DIR   meta.txt: B Hkv G N D scale split dtype ragged
 *                        q.bin [B,Hkv,G,D], k.bin / v.bin [B,Hkv,N,D] (2-byte elements),
 *                        lens.bin int32 [B] (tokens of each sequence) when ragged is 1
 *                        -> out.bin (tc_decode_attention, workspace from hipMalloc)
 *                           out_noalloc.bin (tc_decode_attention_noalloc)
 *   tc_host prefill DIR  meta.txt: B Hq Hkv Q N D scale causal mask_batch dtype
 *                        q.bin [B,Hq,Q,D], k.bin / v.bin [B,Hkv,N,D], mask.bin [mask_batch,Q,N]
 *                        bytes when mask_batch > 0 (its tile map built with tc_prefill_mask_tiles)
 *                        -> out.bin [B,Q,Hq,D] (tc_prefill_attention, splits chosen by the library)
 *   tc_host paged DIR    meta.txt: Hkv G N D scale P pages a c0 c dtype
 *                        q.bin [1,Hkv,G,D], k.bin / v.bin [Hkv,N,D] (one sequence, logical
 *                        order), order.bin int64 [pages] (the order pages are handed out),
 *                        table.bin (D fp32: cos ++ sin of the prune's -(c0 - a) rotation)
 *                        -> tokens in pages order[t / P], slots t % P; when c0 > a a prune
 *                           (tc_page_prune, tc_page_tiles, tc_paged_rotate_keys), then
 *                           tc_decode_paged_attention over the kept tiles: out.bin
 *                           [1,Hkv,G,D], k_pool.bin / v_pool.bin [pages,Hkv,P,D] and
 *                           frags.bin int64 [F,3] (the sequence's fragments)
 *   tc_host splice DIR   meta.txt: L B H cap D a c0 c dtype
 *                        k.bin / v.bin [L,B,H,cap,D], table.bin (D fp32: cos ++ sin)
 *                        -> k_out.bin / v_out.bin (tc_splice_rope over the L layers)
 *
 * Exit status: 0 done, 1 usage or file error, 2 HIP error, 3 the ABI refused
 * the call (its message on stderr). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "threadcut_hip.h"

static char dir_buf[4096];

static const char* path_in(const char* dir, const char* name) {
  snprintf(dir_buf, sizeof dir_buf, "%s/%s", dir, name);
  return dir_buf;
}

static void* read_file(const char* dir, const char* name, size_t bytes) {
  FILE* f = fopen(path_in(dir, name), "rb");
  void* p = malloc(bytes ? bytes : 1);
  if (!f || !p || fread(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "tc_host: cannot read %zu bytes from %s\n", bytes, path_in(dir, name));
    exit(1);
  }
  fclose(f);
  return p;
}

static void write_file(const char* dir, const char* name, const void* p, size_t bytes) {
  FILE* f = fopen(path_in(dir, name), "wb");
  if (!f || fwrite(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "tc_host: cannot write %s\n", path_in(dir, name));
    exit(1);
  }
  fclose(f);
}

static void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "tc_host: %s: %s\n", what, hipGetErrorString(e));
    exit(2);
  }
}

static void abi_ok(int rc, const char* what) {
  if (rc != TC_OK) {
    fprintf(stderr, "tc_host: %s: %s (%s)\n", what, tc_strerror(rc), tc_last_error());
    exit(3);
  }
}

/* A device buffer of `bytes`, filled from `host` unless that is NULL. */
static void* to_device(const void* host, size_t bytes) {
  void* d = NULL;
  hip_ok(hipMalloc(&d, bytes ? bytes : 16), "hipMalloc");
  if (host && bytes) hip_ok(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return d;
}

static int decode(const char* dir) {
  int b, hkv, g, d, split, dtype, ragged;
  long long n;
  float scale;
  FILE* m = fopen(path_in(dir, "meta.txt"), "r");
  if (!m || fscanf(m, "%d %d %d %lld %d %f %d %d %d", &b, &hkv, &g, &n, &d, &scale, &split, &dtype, &ragged) != 9) {
    fprintf(stderr, "tc_host: bad meta.txt\n");
    return 1;
  }
  fclose(m);
  const size_t q_bytes = (size_t)b * hkv * g * d * 2, kv_bytes = (size_t)b * hkv * (size_t)n * d * 2;
  void* q = read_file(dir, "q.bin", q_bytes);
  void* k = read_file(dir, "k.bin", kv_bytes);
  void* v = read_file(dir, "v.bin", kv_bytes);
  void *qd = to_device(q, q_bytes), *kd = to_device(k, kv_bytes), *vd = to_device(v, kv_bytes);
  void *od = to_device(NULL, q_bytes), *od2 = to_device(NULL, q_bytes);
  const int64_t qs[3] = {(int64_t)hkv * g * d, (int64_t)g * d, d};
  const int64_t ks[3] = {(int64_t)hkv * n * d, (int64_t)n * d, d};

  int32_t* lens = ragged ? read_file(dir, "lens.bin", (size_t)b * sizeof(int32_t)) : NULL;
  int32_t* lens_d = ragged ? to_device(lens, (size_t)b * sizeof(int32_t)) : NULL;

  /* The caller sizes the workspace with the library's own split arithmetic. */
  const int splits = tc_decode_num_splits(b, hkv, n, split, ragged);
  if (splits < 0) abi_ok(-splits, "tc_decode_num_splits");
  const size_t ws_bytes = tc_decode_workspace_bytes(b, hkv, g, d, splits);
  void* ws = to_device(NULL, ws_bytes);
  abi_ok(tc_decode_attention(qd, qs, kd, ks, vd, ks, lens_d, n, b, hkv, g, d, dtype, scale, split, ws, ws_bytes,
                             od, qs, NULL),
         "tc_decode_attention");
  abi_ok(tc_decode_attention_noalloc(qd, qs, kd, ks, vd, ks, lens_d, n, b, hkv, g, d, dtype, scale, split, od2, qs,
                                     NULL),
         "tc_decode_attention_noalloc");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");

  void* out = malloc(q_bytes);
  hip_ok(hipMemcpy(out, od, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "out.bin", out, q_bytes);
  hip_ok(hipMemcpy(out, od2, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "out_noalloc.bin", out, q_bytes);
  printf("decode B=%d Hkv=%d G=%d N=%lld splits=%d workspace=%zu\n", b, hkv, g, n, splits, ws_bytes);
  hipFree(qd); hipFree(kd); hipFree(vd); hipFree(od); hipFree(od2); hipFree(ws);
  if (ragged) { hipFree(lens_d); free(lens); }
  free(q); free(k); free(v); free(out);
  return 0;
}

static int prefill(const char* dir) {
  int b, hq, hkv, d, causal, mb, dtype;
  long long ql, n;
  float scale;
  FILE* m = fopen(path_in(dir, "meta.txt"), "r");
  if (!m || fscanf(m, "%d %d %d %lld %lld %d %f %d %d %d", &b, &hq, &hkv, &ql, &n, &d, &scale, &causal, &mb,
                   &dtype) != 10) {
    fprintf(stderr, "tc_host: bad meta.txt\n");
    return 1;
  }
  fclose(m);
  const size_t q_bytes = (size_t)b * hq * (size_t)ql * d * 2, kv_bytes = (size_t)b * hkv * (size_t)n * d * 2;
  void* q = read_file(dir, "q.bin", q_bytes);
  void* k = read_file(dir, "k.bin", kv_bytes);
  void* v = read_file(dir, "v.bin", kv_bytes);
  void *qd = to_device(q, q_bytes), *kd = to_device(k, kv_bytes), *vd = to_device(v, kv_bytes);
  void* od = to_device(NULL, q_bytes);
  const int64_t qs[3] = {(int64_t)hq * ql * d, (int64_t)ql * d, d};
  const int64_t ks[3] = {(int64_t)hkv * n * d, (int64_t)n * d, d};
  const int64_t os[3] = {(int64_t)ql * hq * d, (int64_t)hq * d, d};

  void *mask = NULL, *maskd = NULL, *tilesd = NULL;
  size_t tiles_bytes = 0;
  int64_t ms[3] = {0, 0, 1};
  if (mb > 0) {
    const size_t mask_bytes = (size_t)mb * (size_t)ql * (size_t)n;
    mask = read_file(dir, "mask.bin", mask_bytes);
    maskd = to_device(mask, mask_bytes);
    ms[0] = mb > 1 ? ql * n : 0;  /* one mask for every sequence: batch stride 0 */
    ms[1] = n;
    tiles_bytes = tc_prefill_tiles_bytes(ql, n, mb, hq, hkv);
    if (!tiles_bytes) abi_ok(TC_ERR_INVALID_ARGUMENT, "tc_prefill_tiles_bytes");
    tilesd = to_device(NULL, tiles_bytes);
    abi_ok(tc_prefill_mask_tiles(maskd, ms, mb, ql, n, hq, hkv, tilesd, tiles_bytes, NULL), "tc_prefill_mask_tiles");
  }
  const int splits = tc_prefill_num_splits(b, ql, n, hq, hkv);
  if (splits < 0) abi_ok(-splits, "tc_prefill_num_splits");
  const size_t ws_bytes = tc_prefill_workspace_bytes(b, ql, hq, splits);
  void* ws = to_device(NULL, ws_bytes);
  abi_ok(tc_prefill_attention(qd, qs, kd, ks, vd, ks, maskd, ms, tilesd, tiles_bytes, causal, ql, n, b, hq, hkv, d,
                              dtype, scale, splits, ws, ws_bytes, od, os, NULL),
         "tc_prefill_attention");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  void* out = malloc(q_bytes);
  hip_ok(hipMemcpy(out, od, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "out.bin", out, q_bytes);
  printf("prefill B=%d Hq=%d Hkv=%d Q=%lld N=%lld splits=%d mask_batch=%d causal=%d\n", b, hq, hkv, ql, n, splits,
         mb, causal);
  hipFree(qd); hipFree(kd); hipFree(vd); hipFree(od); hipFree(ws);
  if (maskd) { hipFree(maskd); hipFree(tilesd); free(mask); }
  free(q); free(k); free(v); free(out);
  return 0;
}

static void* upload_tiles(const int64_t* frags, int64_t nf, int64_t page_tokens, int64_t* count) {
  const int64_t nt = tc_page_tiles(frags, nf, page_tokens, 0, NULL, 0);
  if (nt < 0) abi_ok((int)-nt, "tc_page_tiles");
  int32_t* tiles = calloc((size_t)(nt ? nt : 1) * 4, sizeof(int32_t));
  if (nt && tc_page_tiles(frags, nf, page_tokens, 0, tiles, nt) != nt)
    abi_ok(TC_ERR_INVALID_ARGUMENT, "tc_page_tiles");
  void* d = to_device(tiles, (size_t)(nt ? nt : 1) * 4 * sizeof(int32_t));
  free(tiles);
  *count = nt;
  return d;
}

static int paged(const char* dir) {
  int hkv, g, d, pt, pages, dtype;
  long long n, a, c0, c;
  float scale;
  FILE* m = fopen(path_in(dir, "meta.txt"), "r");
  if (!m || fscanf(m, "%d %d %lld %d %f %d %d %lld %lld %lld %d", &hkv, &g, &n, &d, &scale, &pt, &pages, &a, &c0,
                   &c, &dtype) != 11 || n < 1 || pt < 1 || (n + pt - 1) / pt > pages) {
    fprintf(stderr, "tc_host: bad meta.txt\n");
    return 1;
  }
  fclose(m);
  const size_t q_bytes = (size_t)hkv * g * d * 2, seq_bytes = (size_t)hkv * (size_t)n * d * 2;
  const size_t pool_elems = (size_t)pages * hkv * pt * d, row = (size_t)d;
  uint16_t* q = read_file(dir, "q.bin", q_bytes);
  uint16_t* k = read_file(dir, "k.bin", seq_bytes);
  uint16_t* v = read_file(dir, "v.bin", seq_bytes);
  int64_t* order = read_file(dir, "order.bin", (size_t)pages * sizeof(int64_t));

  /* One fragment per page: tokens [i P, (i + 1) P) in page order[i], from slot 0. */
  int64_t nf = (n + pt - 1) / pt;
  int64_t* frags = malloc((size_t)(nf + 1) * 3 * sizeof(int64_t));
  uint16_t* kpool = calloc(pool_elems, 2);
  uint16_t* vpool = calloc(pool_elems, 2);
  for (int64_t i = 0; i < nf; ++i) {
    frags[3 * i] = order[i];
    frags[3 * i + 1] = 0;
    frags[3 * i + 2] = (i + 1) * pt <= n ? pt : n - i * pt;
  }
  for (int64_t t = 0; t < n; ++t)
    for (int h = 0; h < hkv; ++h) {
      const size_t dst = (((size_t)order[t / pt] * hkv + h) * pt + (size_t)(t % pt)) * row;
      memcpy(kpool + dst, k + ((size_t)h * n + t) * row, row * 2);
      memcpy(vpool + dst, v + ((size_t)h * n + t) * row, row * 2);
    }
  void* kd = to_device(kpool, pool_elems * 2);
  void* vd = to_device(vpool, pool_elems * 2);
  const int64_t ps[3] = {(int64_t)hkv * pt * d, (int64_t)pt * d, d};

  if (c0 > a) {
    int64_t* kept = malloc((size_t)(nf + 1) * 3 * sizeof(int64_t));
    int64_t* suffix = malloc((size_t)nf * 3 * sizeof(int64_t));
    int64_t* freed = malloc((size_t)nf * sizeof(int64_t));
    int64_t counts[3];
    abi_ok(tc_page_prune(frags, nf, pt, a, c0, c, kept, suffix, freed, counts), "tc_page_prune");
    int64_t nt = 0;
    void* sd = upload_tiles(suffix, counts[1], pt, &nt);
    float* table = read_file(dir, "table.bin", (size_t)d * sizeof(float));
    void* pools[1] = {kd};
    abi_ok(tc_paged_rotate_keys(pools, 1, ps, pages, pt, sd, nt, hkv, d, dtype, table, NULL),
           "tc_paged_rotate_keys");
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hipFree(sd);
    free(table);
    memcpy(frags, kept, (size_t)counts[0] * 3 * sizeof(int64_t));
    nf = counts[0];
    printf("prune a=%lld c0=%lld c=%lld: %lld fragments kept, %lld pages freed, %lld tiles rotated\n", a, c0, c,
           (long long)counts[0], (long long)counts[2], (long long)nt);
    free(kept); free(suffix); free(freed);
  }

  int64_t mt = 0;
  void* tab = upload_tiles(frags, nf, pt, &mt);
  const int32_t cnt = (int32_t)mt;
  void* cnt_d = to_device(&cnt, sizeof cnt);
  if (mt < 1) mt = 1;  /* the table's width, as the library sizes it */
  const int splits = tc_decode_num_splits(1, hkv, 16 * mt, 0, 0);
  if (splits < 0) abi_ok(-splits, "tc_decode_num_splits");
  const size_t ws_bytes = tc_decode_workspace_bytes(1, hkv, g, d, splits);
  void* ws = to_device(NULL, ws_bytes);
  void* qd = to_device(q, q_bytes);
  void* od = to_device(NULL, q_bytes);
  const int64_t qs[3] = {(int64_t)hkv * g * d, (int64_t)g * d, d};
  abi_ok(tc_decode_paged_attention(qd, qs, kd, vd, ps, pages, pt, tab, cnt_d, mt, 1, hkv, g, d, dtype, scale, 0, ws,
                                   ws_bytes, od, qs, NULL),
         "tc_decode_paged_attention");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  hip_ok(hipMemcpy(q, od, q_bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "out.bin", q, q_bytes);
  hip_ok(hipMemcpy(kpool, kd, pool_elems * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  hip_ok(hipMemcpy(vpool, vd, pool_elems * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "k_pool.bin", kpool, pool_elems * 2);
  write_file(dir, "v_pool.bin", vpool, pool_elems * 2);
  write_file(dir, "frags.bin", frags, (size_t)nf * 3 * sizeof(int64_t));
  printf("paged decode Hkv=%d G=%d tiles=%lld splits=%d\n", hkv, g, (long long)cnt, splits);
  hipFree(kd); hipFree(vd); hipFree(tab); hipFree(cnt_d); hipFree(ws); hipFree(qd); hipFree(od);
  free(q); free(k); free(v); free(order); free(frags); free(kpool); free(vpool);
  return 0;
}

static int splice(const char* dir) {
  int layers, b, h, d, dtype;
  long long cap, a, c0, c;
  FILE* m = fopen(path_in(dir, "meta.txt"), "r");
  if (!m || fscanf(m, "%d %d %d %lld %d %lld %lld %lld %d", &layers, &b, &h, &cap, &d, &a, &c0, &c, &dtype) != 9 ||
      layers < 1 || layers > 64) {
    fprintf(stderr, "tc_host: bad meta.txt\n");
    return 1;
  }
  fclose(m);
  const size_t layer_elems = (size_t)b * h * (size_t)cap * d, bytes = layer_elems * 2 * layers;
  void* k = read_file(dir, "k.bin", bytes);
  void* v = read_file(dir, "v.bin", bytes);
  float* table = read_file(dir, "table.bin", (size_t)d * sizeof(float));
  char *kd = to_device(k, bytes), *vd = to_device(v, bytes);
  void* kp[64];
  void* vp[64];
  for (int l = 0; l < layers; ++l) {
    kp[l] = kd + (size_t)l * layer_elems * 2;
    vp[l] = vd + (size_t)l * layer_elems * 2;
  }
  const int64_t st[3] = {(int64_t)h * cap * d, (int64_t)cap * d, d};
  abi_ok(tc_splice_rope(kp, vp, layers, st, b, h, cap, d, dtype, a, c0, c, table, NULL), "tc_splice_rope");
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  hip_ok(hipMemcpy(k, kd, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  hip_ok(hipMemcpy(v, vd, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  write_file(dir, "k_out.bin", k, bytes);
  write_file(dir, "v_out.bin", v, bytes);
  printf("splice L=%d B=%d H=%d cap=%lld a=%lld c0=%lld c=%lld\n", layers, b, h, cap, a, c0, c);
  hipFree(kd); hipFree(vd);
  free(k); free(v); free(table);
  return 0;
}

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: tc_host decode|prefill|paged|splice DIR\n");
    return 1;
  }
  setvbuf(stdout, NULL, _IONBF, 0);
  if (!strcmp(argv[1], "decode")) return decode(argv[2]);
  if (!strcmp(argv[1], "prefill")) return prefill(argv[2]);
  if (!strcmp(argv[1], "paged")) return paged(argv[2]);
  if (!strcmp(argv[1], "splice")) return splice(argv[2]);
  fprintf(stderr, "tc_host: unknown mode %s\n", argv[1]);
  return 1;
}
