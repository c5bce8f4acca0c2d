// step_cpp.cpp — runs one attention step through the C++ host mirror (include/fqa_step.hpp)
// for tests/test_gpu_cpp_host.py.  Input/output are raw little-endian files:
//   in:  int32 R, T, max_ctx, pool_pages; int32 computed[R], n_new[R], bt_off[R+1],
//        bt_pages[bt_off[R]]; uint16 qkv[T*6144]; float wq[128], wk[128];
//        uint16 pool[pool_pages*8*4096]
//   out: int32 meta[16]; uint16 qkv[T*6144]; uint16 attn[T*4096]
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/fqa_compat.hpp"  // fq::ForwardInput, the reference's batch format
#include "../../include/fqa_step.hpp"

template <class T>
static void rd(FILE* f, T* p, size_t n) {
  if (n && std::fread(p, sizeof(T), n, f) != n) { std::fprintf(stderr, "short read\n"); std::exit(2); }
}

int main(int argc, char** argv) {
  if (argc != 3) { std::fprintf(stderr, "usage: step_cpp in out\n"); return 2; }
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  int32_t hdr[4];
  rd(f, hdr, 4);
  const int R = hdr[0], T = hdr[1], max_ctx = hdr[2];
  const int64_t pool_pages = hdr[3];
  std::vector<int32_t> computed(R), n_new(R), off(R + 1);
  rd(f, computed.data(), R);
  rd(f, n_new.data(), R);
  rd(f, off.data(), R + 1);
  std::vector<int32_t> pages(off[R]);
  rd(f, pages.data(), pages.size());
  // the reference's ForwardInput, filled the way Request::EmitChunk fills it
  fq::ForwardInput in;
  for (int r = 0; r < R; ++r) {
    in.AddRequest(std::vector<int>(pages.begin() + off[r], pages.begin() + off[r + 1]));
    for (int k = 0; k < n_new[r]; ++k) in.AddRow(0, computed[r] + k, r);
  }
  // ... and converted to the mirror's per-request batch the way a binding in
  // ModelRuntime::Forward (model_runtime.cu:304-310) does
  fqa::BatchInput b;
  b.computed.assign(in.block_tables.size(), 0);
  b.n_new.assign(in.block_tables.size(), 0);
  for (int t = 0; t < in.NumRows(); ++t) {
    const int r = in.req_index[t];
    if (b.n_new[r]++ == 0) b.computed[r] = in.positions[t];
  }
  b.block_tables.assign(in.block_tables.begin(), in.block_tables.end());
  std::vector<uint16_t> qkv((size_t)T * 6144);
  std::vector<float> wq(128), wk(128);
  const size_t pool_elems = (size_t)pool_pages * 8 * 4096;
  std::vector<uint16_t> pool(pool_elems);
  rd(f, qkv.data(), qkv.size());
  rd(f, wq.data(), 128);
  rd(f, wk.data(), 128);
  rd(f, pool.data(), pool.size());
  std::fclose(f);

  try {
    hipStream_t s;
    fqa::HipCheck(hipStreamCreate(&s), "stream");
    fqa::StepContext ctx(T, R, max_ctx, pool_pages);
    fqa::DeviceBuffer<uint16_t> d_qkv(qkv.size()), d_pool(pool.size()), d_out((size_t)T * 4096);
    fqa::DeviceBuffer<float> d_wq(128), d_wk(128);
    d_qkv.Upload(qkv.data(), qkv.size(), s);
    d_pool.Upload(pool.data(), pool.size(), s);
    d_wq.Upload(wq.data(), 128, s);
    d_wk.Upload(wk.data(), 128, s);
    fqa::HipCheck(hipMemsetAsync(d_out.D(), 0, (size_t)T * 4096 * 2, s), "memset");
    ctx.PrepareInputs(b, s);
    ctx.RunLayer(d_qkv.D(), d_wq.D(), d_wk.D(), d_pool.D(), d_out.D(), s);
    std::vector<int32_t> meta(16);
    std::vector<uint16_t> out((size_t)T * 4096);
    fqa::HipCheck(hipMemcpyAsync(meta.data(), ctx.Meta(), 64, hipMemcpyDeviceToHost, s), "d2h");
    fqa::HipCheck(hipMemcpyAsync(qkv.data(), d_qkv.D(), qkv.size() * 2, hipMemcpyDeviceToHost, s), "d2h");
    fqa::HipCheck(hipMemcpyAsync(out.data(), d_out.D(), out.size() * 2, hipMemcpyDeviceToHost, s), "d2h");
    fqa::HipCheck(hipStreamSynchronize(s), "sync");
    FILE* g = std::fopen(argv[2], "wb");
    std::fwrite(meta.data(), 4, 16, g);
    std::fwrite(qkv.data(), 2, qkv.size(), g);
    std::fwrite(out.data(), 2, out.size(), g);
    std::fclose(g);
    (void)hipStreamDestroy(s);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "step_cpp: %s\n", e.what());
    return 1;
  }
  return 0;
}
