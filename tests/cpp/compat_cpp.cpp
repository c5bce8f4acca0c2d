// compat_cpp.cpp — the reference engine's attention section of ModelRuntime::RunLayersBody
// (engine/src/model_runtime.cu:263-278), with StepContext::PrepareInputs (:295-302) before
// it, written against include/fqa_compat.hpp with the reference's own call expressions.
// For tests/test_gpu_compat.py.  Raw little-endian files:
//   in:  int32 R, T, max_ctx, pool_pages, layers; int32 computed[R], n_new[R], bt_off[R+1],
//        bt_pages[bt_off[R]]; uint16 qkv[layers][T*6144]; float wq[128], wk[128];
//        uint16 pool[layers][pool_pages*8*4096]
//   out: uint16 qkv[layers][T*6144]; uint16 attn[layers][T*4096];
//        uint16 pool[layers][pool_pages*8*4096]; int32 n_decode, n_prefill, prefill_max_qlen
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/fqa_compat.hpp"

// The fields of the reference's ModelSpec (model_spec.h:10-26) the path reads.
struct Spec {
  int hidden_size = 4096, num_layers = 2, num_heads = 32, num_kv_heads = 8, head_dim = 128;
  float rms_eps = 1e-6f, rope_theta = 1000000.0f;
  int QDim() const { return num_heads * head_dim; }
  int KvDim() const { return num_kv_heads * head_dim; }
};

template <class T>
static void rd(FILE* f, T* p, size_t n) {
  if (n && std::fread(p, sizeof(T), n, f) != n) { std::fprintf(stderr, "short read\n"); std::exit(2); }
}

int main(int argc, char** argv) {
  if (argc != 3) { std::fprintf(stderr, "usage: compat_cpp in out\n"); return 2; }
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  int32_t hdr[5];
  rd(f, hdr, 5);
  const int R = hdr[0], T = hdr[1], max_ctx = hdr[2], pool_pages = hdr[3], L = hdr[4];
  std::vector<int32_t> computed(R), n_new(R), off(R + 1);
  rd(f, computed.data(), R);
  rd(f, n_new.data(), R);
  rd(f, off.data(), R + 1);
  std::vector<int32_t> pages(off[R]);
  rd(f, pages.data(), pages.size());
  const size_t qkv_elems = (size_t)T * 6144, pool_elems = (size_t)pool_pages * 8 * 4096;
  std::vector<uint16_t> qkv(qkv_elems * L), pool(pool_elems * L);
  std::vector<float> wq(128), wk(128);
  rd(f, qkv.data(), qkv.size());
  rd(f, wq.data(), 128);
  rd(f, wk.data(), 128);
  rd(f, pool.data(), pool.size());
  std::fclose(f);

  // ForwardInput as the scheduler's EmitChunk fills it (scheduler.h:66-72)
  fq::ForwardInput in;
  for (int r = 0; r < R; ++r) {
    in.AddRequest(std::vector<int>(pages.begin() + off[r], pages.begin() + off[r + 1]));
    for (int k = 0; k < n_new[r]; ++k) in.AddRow(1000 + r, computed[r] + k, r);
    in.SampleLastRow(fq::SampleParams{0.7f, 0.9f});
  }

  try {
    Spec spec;
    spec.num_layers = L;
    hipStream_t stream;
    fqa::HipCheck(hipStreamCreate(&stream), "stream");
    fq::StepContext ctx_(T, R, max_ctx);
    fq::KvStore store(spec, (int64_t)pool_pages);
    fq::KvStore* store_ = &store;
    fq::RopeTables rope;
    rope.Build(spec, max_ctx);
    fqa::DeviceBuffer<uint16_t> qkv_d(qkv_elems), attn_d((size_t)T * 4096);
    fqa::DeviceBuffer<float> q_norm(128), k_norm(128);
    // the reference's decode partials (RuntimeBuffers, model_runtime.cu:191-194); unused here
    fqa::DeviceBuffer<float> dec_pm(16), dec_pl(16), dec_pa(16);
    q_norm.Upload(wq.data(), 128, stream);
    k_norm.Upload(wk.data(), 128, stream);
    for (int l = 0; l < L; ++l)
      fqa::HipCheck(hipMemcpyAsync(store.KV(l), pool.data() + l * pool_elems, pool_elems * 2,
                                   hipMemcpyHostToDevice, stream), "pool upload");

    std::mt19937 rng(7);
    ctx_.PrepareInputs(in, rng, stream);

    const int n_rows = ctx_.n_rows;
    const int n_heads = spec.num_heads, n_kv = spec.num_kv_heads, head_dim = spec.head_dim;
    const int qkv_dim = spec.QDim() + 2 * spec.KvDim();
    const float eps = spec.rms_eps, scale = 1.0f / std::sqrt(static_cast<float>(head_dim));
    const int block_size = store_->BlockSize();
    fq::bf16* qkv_b = reinterpret_cast<fq::bf16*>(qkv_d.D());
    fq::bf16* attn_b = reinterpret_cast<fq::bf16*>(attn_d.D());
    std::vector<uint16_t> out_qkv(qkv_elems * L), out_attn((size_t)T * 4096 * L);
    for (int l = 0; l < L; ++l) {
      // stands for LaunchGemm(..., buf_.qkv.D(), ...) of model_runtime.cu:261
      qkv_d.Upload(qkv.data() + l * qkv_elems, qkv_elems, stream);
      fqa::HipCheck(hipMemsetAsync(attn_d.D(), 0, (size_t)T * 4096 * 2, stream), "memset");
      // model_runtime.cu:263-278, verbatim up to the buffer names
      fq::LaunchHeadNormRope(qkv_b, q_norm.D(), k_norm.D(), rope.Cos(), rope.Sin(),
                             ctx_.pos.D(), n_rows, n_heads, n_kv, head_dim, qkv_dim, eps, stream);
      store_->StoreKV(l, qkv_b, ctx_.bt.D(), ctx_.bt_stride, ctx_.req.D(), ctx_.pos.D(), n_rows,
                      stream);
      fq::LaunchAttnDecodeCute(qkv_b, qkv_dim, store_->KV(l), attn_b, n_heads, n_kv, head_dim,
                               ctx_.pos.D(), ctx_.qstart.D(), ctx_.decode_rids.D(),
                               ctx_.n_decode, ctx_.bt.D(), ctx_.bt_stride, block_size, scale,
                               dec_pm.D(), dec_pl.D(), dec_pa.D(), stream);
      fq::LaunchAttnPrefillCute(qkv_b, qkv_dim, store_->KV(l), attn_b, n_heads, n_kv, head_dim,
                                ctx_.pos.D(), ctx_.qstart.D(), ctx_.qlen.D(),
                                ctx_.prefill_rids.D(), ctx_.n_prefill, ctx_.prefill_max_qlen,
                                ctx_.bt.D(), ctx_.bt_stride, block_size, scale, stream);
      fqa::HipCheck(hipMemcpyAsync(out_qkv.data() + l * qkv_elems, qkv_d.D(), qkv_elems * 2,
                                   hipMemcpyDeviceToHost, stream), "d2h");
      fqa::HipCheck(hipMemcpyAsync(out_attn.data() + l * (size_t)T * 4096, attn_d.D(),
                                   (size_t)T * 4096 * 2, hipMemcpyDeviceToHost, stream), "d2h");
      fqa::HipCheck(hipStreamSynchronize(stream), "sync");
    }
    for (int l = 0; l < L; ++l)
      fqa::HipCheck(hipMemcpyAsync(pool.data() + l * pool_elems, store.KV(l), pool_elems * 2,
                                   hipMemcpyDeviceToHost, stream), "d2h");
    fqa::HipCheck(hipStreamSynchronize(stream), "sync");
    FILE* g = std::fopen(argv[2], "wb");
    std::fwrite(out_qkv.data(), 2, out_qkv.size(), g);
    std::fwrite(out_attn.data(), 2, out_attn.size(), g);
    std::fwrite(pool.data(), 2, pool.size(), g);
    const int32_t counts[3] = {ctx_.n_decode, ctx_.n_prefill, ctx_.prefill_max_qlen};
    std::fwrite(counts, 4, 3, g);
    std::fclose(g);
    (void)hipStreamDestroy(stream);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "compat_cpp: %s\n", e.what());
    return 1;
  }
  return 0;
}
