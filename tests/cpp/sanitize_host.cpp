// sanitize_host.cpp — the host C++ of the library under AddressSanitizer +
// UndefinedBehaviorSanitizer (tests/test_sanitize.py), with the device stubbed out:
//  * flashqwen_amd/csrc/fqa_host.cpp (RoPE tables, pool sizing) linked in as it is;
//  * include/fqa_compat.hpp's StepContext::PrepareInputs, RopeTables::Build and KvStore
//    sizing, over stub HIP entry points that keep "device" buffers in host memory, and a
//    stub fqa_pack that runs the CPU oracle's pack (oracle/fqa_oracle.c) on them, so the
//    packed arrays can be checked against the oracle called directly;
//  * the compat header's rejections (ragged rows, unknown request, too many rows) throw.
// Host code only: nothing here touches a GPU.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "../../include/fqa_compat.hpp"
#include "../../oracle/fqa_oracle.h"

// ---- stub HIP runtime: "device" memory is host memory, copies are memcpy -------------
static size_t g_live = 0;  // outstanding stub allocations
hipError_t hipMalloc(void** p, size_t n) {
  *p = std::malloc(n ? n : 1);
  ++g_live;
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void* p) {
  if (p) --g_live;
  std::free(p);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t) {
  std::memcpy(dst, src, n);
  return hipSuccess;
}
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipMemGetInfo(size_t* freeb, size_t* totalb) {
  *totalb = 256ull << 20;  // a small device (the stub pool is host memory): 64 MiB in use
  *freeb = *totalb - (64ull << 20);
  return hipSuccess;
}
const char* hipGetErrorString(hipError_t) { return "stub"; }

// ---- stub library entry points the headers reference ----------------------------------
extern "C" {
int32_t fqa_dec_default_waves(int32_t) { return 1024; }
int32_t fqa_dec_wave_bound(int32_t, int32_t waves) { return waves > 0 ? waves : 0; }
int32_t fqa_pre_item_bound(int32_t n_reqs, int32_t max_rows, int32_t tile) {
  return max_rows / tile + n_reqs;
}
int64_t fqa_decode_workspace_bytes(const fqa_dims*, int32_t waves) {
  return (int64_t)waves * 2 * 4 * (2 + 128) * 4;
}
int g_rope_rows = -1;  // rope_max_pos of the last fqa_qknorm_rope call
int fqa_qknorm_rope(const fqa_dims*, uint16_t*, const float*, const float*, const float*,
                    const float*, int32_t rope_max_pos, const int32_t*, const int32_t*, int32_t,
                    void*) {
  g_rope_rows = rope_max_pos;
  return FQA_OK;
}
// fqa_pack on host memory: the oracle's pack, with the arguments fqa.h gives it
int fqa_pack(const fqa_batch* b, const fqa_pack_cfg* c, const fqa_pack_out* o, void*) {
  fqo_pack(b->n_reqs, b->computed, b->n_new, b->bt_off, b->bt_pages, c->max_rows,
           c->max_blocks, c->pool_pages, c->dec_grid_waves, c->dec_min_pages, c->dec_wave_cap,
           c->pre_tile_q, c->pre_item_cap, c->dec_share, c->dec_prefix_pages, c->dec_pre_cap,
           o->cu_seqlens, o->qlen, o->positions, o->row_req, o->slot_mapping, o->block_tables,
           o->decode_rids, o->prefill_rids, o->dec_seqs, o->dec_waves, o->pre_items,
           o->dec_prefix, o->dec_pre_items, o->meta);
  return FQA_OK;
}
}

static int failures = 0;
#define EXPECT(cond, what)                      \
  do {                                          \
    if (!(cond)) {                              \
      std::fprintf(stderr, "FAIL: %s\n", what); \
      ++failures;                               \
    }                                           \
  } while (0)

struct Spec {  // the ModelSpec fields the compat classes read (model_spec.h:11-19)
  int num_layers = 2, num_heads = 32, num_kv_heads = 8, head_dim = 128;
  float rope_theta = 1e6f, rms_eps = 1e-6f;
};

template <class F>
static bool Throws(F f) {
  try {
    f();
  } catch (const std::runtime_error&) {
    return true;
  }
  return false;
}

// A batch as Request::EmitChunk emits it: request r's rows at positions computed..
static fq::ForwardInput MakeInput(std::mt19937& g, int R, int max_ctx, std::vector<int>& comp,
                                  std::vector<int>& nnew) {
  fq::ForwardInput in;
  int next_page = 0;
  comp.assign(R, 0);
  nnew.assign(R, 0);
  for (int r = 0; r < R; ++r) {
    comp[r] = (int)(g() % (max_ctx / 2));
    nnew[r] = g() % 3 ? 1 : 1 + (int)(g() % 70);
    std::vector<int> table((comp[r] + nnew[r] + 15) / 16);
    for (auto& p : table) p = next_page++;
    const int rr = in.AddRequest(table);
    for (int k = 0; k < nnew[r]; ++k) in.AddRow((int)(g() % 50000), comp[r] + k, rr);
    in.SampleLastRow({0.7f, 0.9f});
  }
  return in;
}

int main() {
  // fqa_host.cpp: RoPE tables bit-identical to the oracle's restatement of RopeTables::Build
  {
    const int P = 64;
    std::vector<float> c(P * 64), s(P * 64), oc(P * 64), os(P * 64);
    EXPECT(fqa_rope_tables(P, 128, 1e6f, c.data(), s.data()) == FQA_OK, "rope tables");
    fqo_rope_tables(P, 128, 1e6f, oc.data(), os.data());
    EXPECT(!std::memcmp(c.data(), oc.data(), c.size() * 4) &&
               !std::memcmp(s.data(), os.data(), s.size() * 4),
           "rope tables differ from the oracle's");
    EXPECT(fqa_rope_tables(-1, 128, 1e6f, c.data(), s.data()) == FQA_EINVAL, "rope EINVAL");
  }
  // fqa_host.cpp: pool sizing
  {
    const fqa_dims d{32, 8, 128, 16, 6144, 1e-6f, 0.f};
    EXPECT(fqa_pool_bytes(&d, 3) == 3LL * 8 * 2 * 16 * 128 * 2, "pool bytes");
    int64_t pages = -1;
    EXPECT(fqa_pool_pages(&d, 288ull << 30, 8ull << 30, 0.9f, 36, 32768, &pages) == FQA_OK,
           "pool pages");
    EXPECT(pages > 0, "pool pages > 0");
    EXPECT(fqa_pool_pages(&d, 1ull << 20, 0, 0.9f, 36, 32768, &pages) == FQA_ENOSPACE,
           "pool ENOSPACE");
    int64_t want = -1;
    fqa_pool_pages(&d, 256ull << 20, 64ull << 20, 0.9f, 2, 4096, &want);
    EXPECT(fqa_pool_pages_device(&d, 0.9f, 2, 4096, &pages) == FQA_OK && pages == want,
           "device pool pages from hipMemGetInfo");
  }
  // fqa_compat.hpp over the stubs
  {
    Spec spec;
    fq::RopeTables rope;
    rope.Build(spec, 512);
    EXPECT(rope.Cos()[64] == std::cos(1.0f), "RopeTables row 1, dim 0");
    fq::KvStore kv(spec, 4096, 0.9f);  // sized from the stub's free memory
    EXPECT(kv.NumBlocks() == (int)(((uint64_t)(0.9f * (float)(256ull << 20)) - (64ull << 20)) /
                                   (2ull * 2 * 16 * 8 * 128 * 2)),
           "KvStore pages from free memory");
    EXPECT(Throws([&] { fq::KvStore k3(spec, 1 << 20, 0.9f); }), "KvStore: no room for max_ctx");
    fq::KvStore kv2(spec, (int64_t)64);
    EXPECT(kv2.NumBlocks() == 64, "KvStore explicit pages");

    std::mt19937 g(123), rng(7);
    for (int trial = 0; trial < 20; ++trial) {
      const int R = 1 + (int)(g() % 40), max_ctx = 2048;
      std::vector<int> comp, nnew;
      fq::ForwardInput in = MakeInput(g, R, max_ctx, comp, nnew);
      fq::StepContext ctx(in.NumRows() + 4, 64, max_ctx);
      hipStream_t s = reinterpret_cast<hipStream_t>(0x100 + trial);
      ctx.PrepareInputs(in, rng, s);
      int nd = 0, np = 0, mq = 1;
      for (int r = 0; r < R; ++r) {
        if (nnew[r] == 1) ++nd;
        else ++np, mq = std::max(mq, nnew[r]);
      }
      EXPECT(ctx.n_rows == in.NumRows() && ctx.n_decode == nd && ctx.n_prefill == np &&
                 ctx.prefill_max_qlen == mq && ctx.n_sample == R,
             "PrepareInputs host counts");
      // the packed arrays against the oracle's pack of the same batch
      std::vector<int32_t> off(R + 1, 0), pages;
      for (int r = 0; r < R; ++r) {
        pages.insert(pages.end(), in.block_tables[r].begin(), in.block_tables[r].end());
        off[r + 1] = (int32_t)pages.size();
      }
      const int T = in.NumRows(), mb = ctx.max_blocks;
      std::vector<int32_t> cu(R + 1), ql(R), pos(T), req(T), slot(T), bt((size_t)R * mb),
          dr(R), pr(R), ds((size_t)R * 4), dw((size_t)ctx.DecWaveCap() * 8),
          it((size_t)ctx.PreItemCap() * 4), meta(16);
      fqo_pack(R, comp.data(), nnew.data(), off.data(), pages.empty() ? off.data() : pages.data(),
               T + 4, mb, 0x7fffffff, 1024, 8, ctx.DecWaveCap(), FQA_PRE_TILE_Q,
               ctx.PreItemCap(), 0, 0, 0, cu.data(), ql.data(), pos.data(), req.data(),
               slot.data(), bt.data(), dr.data(), pr.data(), ds.data(), dw.data(), it.data(),
               nullptr, nullptr, meta.data());
      EXPECT(!std::memcmp(meta.data(), ctx.Meta(), 16 * 4), "meta");
      EXPECT(!std::memcmp(pos.data(), ctx.pos.D(), T * 4), "positions");
      EXPECT(!std::memcmp(slot.data(), ctx.SlotMapping(), T * 4), "slot mapping");
      EXPECT(!std::memcmp(bt.data(), ctx.bt.D(), bt.size() * 4), "block tables");
      EXPECT(!std::memcmp(cu.data(), ctx.qstart.D(), (R + 1) * 4), "cu_seqlens");
    }
    // LaunchHeadNormRope bounds positions by the rows of the table it is given
    {
      std::vector<int> comp, nnew;
      fq::ForwardInput in = MakeInput(g, 3, 2048, comp, nnew);
      fq::StepContext ctx(in.NumRows(), 8, 2048);
      hipStream_t s = reinterpret_cast<hipStream_t>(0x900);
      ctx.PrepareInputs(in, rng, s);
      fq::LaunchHeadNormRope(nullptr, nullptr, nullptr, rope.Cos(), rope.Sin(), ctx.pos.D(),
                             ctx.n_rows, 32, 8, 128, 6144, 1e-6f, s);
      EXPECT(g_rope_rows == 512, "rope rows of a RopeTables");
      std::vector<float> own(64);
      fq::LaunchHeadNormRope(nullptr, nullptr, nullptr, own.data(), own.data(), ctx.pos.D(),
                             ctx.n_rows, 32, 8, 128, 6144, 1e-6f, s);
      EXPECT(g_rope_rows == 2048, "rope rows of a table built elsewhere: max_ctx");
    }
    // rejections
    fq::StepContext ctx(8, 4, 256);
    std::mt19937 r2(1);
    fq::ForwardInput bad;
    bad.AddRequest({0});
    bad.AddRow(1, 0, 0);
    bad.AddRow(2, 5, 0);  // positions not consecutive
    EXPECT(Throws([&] { ctx.PrepareInputs(bad, r2, nullptr); }), "non-consecutive positions");
    fq::ForwardInput unk;
    unk.AddRequest({0});
    unk.AddRow(1, 0, 3);  // unknown request
    EXPECT(Throws([&] { ctx.PrepareInputs(unk, r2, nullptr); }), "unknown request");
    fq::ForwardInput big;
    big.AddRequest({0});
    for (int k = 0; k < 9; ++k) big.AddRow(1, k, 0);  // more rows than the context holds
    EXPECT(Throws([&] { ctx.PrepareInputs(big, r2, nullptr); }), "too many rows");
    EXPECT(Throws([] { fq::StepContext(0, 4, 256); }), "bad StepContext sizes");
  }
  EXPECT(g_live == 0, "stub allocations leaked");
  if (failures) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
