// extern "C" boundary (include/fhecore.h): handle management, argument and
// shape validation, and translation of C++ exceptions into status codes plus
// a thread-local message.  No exception crosses this file's functions.
#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fhecore.h"
#include "ops.hpp"
#include "params.hpp"
#include "sampling.hpp"

// Every handle shares ownership of its context, so handles may be released
// in any order (a garbage collector may finalise a context before its polys).
struct fhe_context {
  std::shared_ptr<fhe::Context> own;
  fhe::Context* c;
};

struct fhe_poly {
  std::shared_ptr<fhe::Context> own;
  fhe::Context* c;
  uint32_t npoly, nlimb;
  uint64_t* data;
  size_t bytes;
};

struct fhe_key {
  std::shared_ptr<fhe::Context> own;
  fhe::Context* c;
  uint64_t* data;  // [dnum][2][L+K][N], Montgomery form
  size_t bytes;
};

namespace {

thread_local std::string g_err;

template <typename F>
int guard(F&& f) {
  try {
    f();
    return FHE_OK;
  } catch (const fhe::ArgError& e) {
    g_err = e.what();
    return FHE_ERR_ARG;
  } catch (const fhe::HipError& e) {
    g_err = e.what();
    return FHE_ERR_HIP;
  } catch (const fhe::StateError& e) {
    g_err = e.what();
    return FHE_ERR_STATE;
  } catch (const std::out_of_range& e) {
    g_err = e.what();
    return FHE_ERR_RANGE;
  } catch (const std::exception& e) {
    g_err = e.what();
    return FHE_ERR_INTERNAL;
  } catch (...) {
    g_err = "unknown error";
    return FHE_ERR_INTERNAL;
  }
}

void need(bool ok, const char* msg) {
  if (!ok) throw fhe::ArgError(msg);
}

size_t words(const fhe::Context& c, uint32_t npoly, uint32_t nlimb) {
  return (size_t)npoly * nlimb * c.n;
}

// (Re)shape a poly handle; storage is reused when the size does not change.
void reshape(fhe_poly* p, uint32_t npoly, uint32_t nlimb) {
  const size_t bytes = words(*p->c, npoly, nlimb) * 8;
  if (bytes != p->bytes) {
    if (p->data) p->c->release(p->data, p->bytes);
    p->data = bytes ? (uint64_t*)p->c->alloc(bytes) : nullptr;
    p->bytes = bytes;
  }
  p->npoly = npoly;
  p->nlimb = nlimb;
}

void same_ctx(const fhe_poly* a, const fhe_poly* b) {
  need(a && b && a->c == b->c, "polys belong to different contexts");
}

// Resolve an output handle that may alias an input: the input's storage is
// read by the launched kernels before (elementwise) or only through scratch.
void prepare_out(fhe_poly* out, uint32_t npoly, uint32_t nlimb) {
  if (out->npoly != npoly || out->nlimb != nlimb) reshape(out, npoly, nlimb);
}

// Writes a result of shape (npoly, nlimb) into `out` through f(dst), where
// `in` is an input that f reads.  If out is that input, the result goes to
// fresh pool storage which then replaces out's: the old storage returns to
// the pool once the launches that read it are queued (the pool is stream
// ordered), so no copy back is needed.
template <class F>
void write_result(fhe_poly* out, const fhe_poly* in, uint32_t npoly, uint32_t nlimb, F&& f) {
  if (out != in) {
    prepare_out(out, npoly, nlimb);
    f(out->data);
    return;
  }
  fhe::Context& c = *out->c;
  const size_t bytes = words(c, npoly, nlimb) * 8;
  uint64_t* fresh = static_cast<uint64_t*>(c.alloc(bytes));
  try {
    f(fresh);
  } catch (...) {
    c.release(fresh, bytes);
    throw;
  }
  if (out->data) c.release(out->data, out->bytes);
  out->data = fresh;
  out->bytes = bytes;
  out->npoly = npoly;
  out->nlimb = nlimb;
}

fhe_key* new_key(const std::shared_ptr<fhe::Context>& own) {
  fhe::Context& c = *own;
  fhe_key* k = new fhe_key;
  k->own = own;
  k->c = &c;
  k->bytes = (size_t)c.dnum * 2 * (c.L + c.K) * c.n * 8;
  k->data = (uint64_t*)c.alloc(k->bytes);
  return k;
}

}  // namespace

extern "C" {

const char* fhe_last_error(void) { return g_err.c_str(); }
int fhe_abi_version(void) { return 1; }

int fhe_gen_moduli(uint32_t log_n, uint32_t depth, uint32_t scale_bits, uint32_t first_bits,
                   uint32_t dnum, uint64_t* q_out, uint64_t* p_out, uint32_t p_cap,
                   uint32_t* num_p) {
  return guard([&] {
    need(q_out && p_out && num_p, "null output");
    need(log_n >= 4 && log_n <= 17, "log_n must be in [4, 17]");
    need(dnum >= 1 && depth + 1 <= 64, "bad depth or dnum");
    need(scale_bits >= 20 && scale_bits <= 60 && first_bits >= 20 && first_bits <= 60,
         "modulus sizes must be in [20, 60] bits");
    std::vector<uint64_t> p;
    const std::vector<uint64_t> q = fhe::gen_moduli(log_n, depth, scale_bits, first_bits, dnum, p);
    need(p.size() <= p_cap, "p_out too small");
    std::memcpy(q_out, q.data(), q.size() * 8);
    std::memcpy(p_out, p.data(), p.size() * 8);
    *num_p = (uint32_t)p.size();
  });
}

int fhe_context_create(uint32_t log_n, const uint64_t* q, uint32_t num_q, const uint64_t* p,
                       uint32_t num_p, uint32_t dnum, int device, fhe_context** out) {
  return guard([&] {
    need(q && out && (p || num_p == 0), "null argument");
    *out = nullptr;
    std::shared_ptr<fhe::Context> c =
        std::make_shared<fhe::Context>(log_n, q, num_q, p, num_p, dnum, device);
    *out = new fhe_context{c, c.get()};
  });
}

int fhe_context_destroy(fhe_context* ctx) {
  return guard([&] {
    if (!ctx) return;
    delete ctx;
  });
}

int fhe_context_info(const fhe_context* ctx, uint32_t* info5) {
  return guard([&] {
    need(ctx && info5, "null argument");
    const fhe::Context& c = *ctx->c;
    info5[0] = c.log_n;
    info5[1] = c.L;
    info5[2] = c.K;
    info5[3] = c.dnum;
    info5[4] = c.alpha;
  });
}

int fhe_alloc_count(uint64_t* count) {
  return guard([&] {
    need(count, "null argument");
    *count = fhe::alloc_requests();
  });
}

int fhe_context_moduli(const fhe_context* ctx, uint64_t* mods, uint64_t* psi) {
  return guard([&] {
    need(ctx, "null context");
    const fhe::Context& c = *ctx->c;
    if (mods) std::memcpy(mods, c.mods.data(), c.mods.size() * 8);
    if (psi) std::memcpy(psi, c.psi.data(), c.psi.size() * 8);
  });
}

int fhe_context_set_stream(fhe_context* ctx, void* hip_stream) {
  return guard([&] {
    need(ctx, "null context");
    fhe::Context& c = *ctx->c;
    fhe::hip_check(hipStreamSynchronize(c.stream), "stream switch");
    hipStream_t s = reinterpret_cast<hipStream_t>(hip_stream);
    if (!s) {
      need(c.own_stream, "context has no own stream");
      return;
    }
    if (c.own_stream) {
      hipStreamDestroy(c.stream);
      c.own_stream = false;
    }
    c.stream = s;
  });
}

int fhe_sync(fhe_context* ctx) {
  return guard([&] {
    need(ctx, "null context");
    fhe::hip_check(hipStreamSynchronize(ctx->c->stream), "fhe_sync");
  });
}

int fhe_profile_begin(fhe_context* ctx) {
  return guard([&] {
    need(ctx, "null context");
    ctx->c->prof.clear();
    ctx->c->prof.on = true;
  });
}

int fhe_profile_end(fhe_context* ctx, char* buf, size_t cap) {
  return guard([&] {
    need(ctx && buf && cap > 2, "null argument");
    fhe::Context& c = *ctx->c;
    fhe::hip_check(hipStreamSynchronize(c.stream), "profile sync");
    std::map<std::string, std::pair<long, double>> agg;
    for (auto& r : c.prof.recs) {
      float ms = 0;
      fhe::hip_check(hipEventElapsedTime(&ms, r.a, r.b), "hipEventElapsedTime");
      auto& e = agg[r.name];
      e.first += 1;
      e.second += ms;
    }
    c.prof.clear();
    c.prof.on = false;
    std::string js = "{";
    bool first = true;
    for (auto& kv : agg) {
      if (!first) js += ",";
      first = false;
      js += "\"" + kv.first + "\":[" + std::to_string(kv.second.first) + "," +
            std::to_string(kv.second.second) + "]";
    }
    js += "}";
    need(js.size() + 1 <= cap, "profile buffer too small");
    std::memcpy(buf, js.c_str(), js.size() + 1);
  });
}

int fhe_ntt_forward(fhe_context* ctx, uint64_t* data, uint32_t npoly, uint32_t nlimb,
                    uint32_t limb0) {
  return guard([&] {
    need(ctx && data, "null argument");
    fhe::Context& c = *ctx->c;
    need(limb0 + nlimb <= c.L + c.K, "limb range exceeds the moduli");
    fhe::ntt_forward(c, data, npoly, (size_t)nlimb * c.n, nlimb, fhe::LimbMap::contiguous(limb0));
  });
}

int fhe_ntt_inverse(fhe_context* ctx, uint64_t* data, uint32_t npoly, uint32_t nlimb,
                    uint32_t limb0) {
  return guard([&] {
    need(ctx && data, "null argument");
    fhe::Context& c = *ctx->c;
    need(limb0 + nlimb <= c.L + c.K, "limb range exceeds the moduli");
    fhe::ntt_inverse(c, data, npoly, (size_t)nlimb * c.n, nlimb, fhe::LimbMap::contiguous(limb0));
  });
}

int fhe_mac(fhe_context* ctx, const uint64_t* x, const uint64_t* w, uint32_t n, uint32_t nq,
            uint64_t* acc) {
  return guard([&] {
    need(ctx && x && w && acc, "null argument");
    need(nq >= 1 && nq <= ctx->c->L, "bad limb count");
    fhe::poly_mac(*ctx->c, acc, x, w, n, nq);
  });
}

int fhe_poly_create(fhe_context* ctx, uint32_t npoly, uint32_t nlimb, fhe_poly** out) {
  return guard([&] {
    need(ctx && out, "null argument");
    need(nlimb <= ctx->c->L + ctx->c->K && npoly <= 65535, "bad poly shape");
    fhe_poly* p = new fhe_poly{ctx->own, ctx->c, 0, 0, nullptr, 0};
    try {
      reshape(p, npoly, nlimb);
    } catch (...) {
      delete p;
      throw;
    }
    *out = p;
  });
}

int fhe_poly_destroy(fhe_poly* p) {
  return guard([&] {
    if (!p) return;
    if (p->data) p->c->release(p->data, p->bytes);
    delete p;
  });
}

int fhe_poly_shape(const fhe_poly* p, uint32_t* npoly, uint32_t* nlimb) {
  return guard([&] {
    need(p && npoly && nlimb, "null argument");
    *npoly = p->npoly;
    *nlimb = p->nlimb;
  });
}

int fhe_poly_data(const fhe_poly* p, uint64_t** dev) {
  return guard([&] {
    need(p && dev, "null argument");
    *dev = p->data;
  });
}

int fhe_poly_upload(fhe_poly* p, const uint64_t* host, uint32_t npoly, uint32_t nlimb) {
  return guard([&] {
    need(p && host, "null argument");
    need(nlimb <= p->c->L + p->c->K, "bad limb count");
    reshape(p, npoly, nlimb);
    fhe::hip_check(hipMemcpyAsync(p->data, host, p->bytes, hipMemcpyHostToDevice, p->c->stream),
                   "upload");
    fhe::hip_check(hipStreamSynchronize(p->c->stream), "upload sync");
  });
}

int fhe_poly_download(const fhe_poly* p, uint64_t* host) {
  return guard([&] {
    need(p && host, "null argument");
    fhe::hip_check(hipMemcpyAsync(host, p->data, p->bytes, hipMemcpyDeviceToHost, p->c->stream),
                   "download");
    fhe::hip_check(hipStreamSynchronize(p->c->stream), "download sync");
  });
}

int fhe_poly_copy(fhe_poly* dst, const fhe_poly* src) {
  return guard([&] {
    same_ctx(dst, src);
    if (dst == src) return;
    reshape(dst, src->npoly, src->nlimb);
    fhe::hip_check(hipMemcpyAsync(dst->data, src->data, src->bytes, hipMemcpyDeviceToDevice,
                                  src->c->stream),
                   "copy");
  });
}

int fhe_drop_limbs(fhe_poly* out, const fhe_poly* a, uint32_t nlimb) {
  return guard([&] {
    same_ctx(out, a);
    need(nlimb >= 1 && nlimb <= a->nlimb, "can only drop limbs");
    fhe::Context& c = *a->c;
    if (out == a && nlimb == a->nlimb) return;
    const uint32_t npoly = a->npoly, nl = a->nlimb;
    const uint64_t* src = a->data;
    write_result(out, a, npoly, nlimb, [&](uint64_t* dst) {
      fhe::poly_copy_limbs(c, dst, nlimb, src, nl, npoly, nlimb);
    });
  });
}

static int binary(fhe_poly* out, const fhe_poly* a, const fhe_poly* b, fhe::BinOp op) {
  return guard([&] {
    same_ctx(a, b);
    same_ctx(out, a);
    need(a->npoly == b->npoly && a->nlimb == b->nlimb, "shape mismatch");
    prepare_out(out, a->npoly, a->nlimb);
    fhe::poly_binary(*a->c, op, out->data, a->data, b->data, a->npoly, a->nlimb);
  });
}

int fhe_add(fhe_poly* out, const fhe_poly* a, const fhe_poly* b) {
  return binary(out, a, b, fhe::OP_ADD);
}
int fhe_sub(fhe_poly* out, const fhe_poly* a, const fhe_poly* b) {
  return binary(out, a, b, fhe::OP_SUB);
}

int fhe_negate(fhe_poly* out, const fhe_poly* a) {
  return guard([&] {
    same_ctx(out, a);
    prepare_out(out, a->npoly, a->nlimb);
    fhe::poly_negate(*a->c, out->data, a->data, a->npoly, a->nlimb);
  });
}

int fhe_mul_plain(fhe_poly* out, const fhe_poly* ct, const fhe_poly* pt) {
  return guard([&] {
    same_ctx(ct, pt);
    same_ctx(out, ct);
    need(pt->npoly == 1 && pt->nlimb >= ct->nlimb, "plaintext must be one poly at >= limbs");
    // Reshaping the plaintext's own handle would free it before it is read.
    need(out != pt || (ct->npoly == 1 && ct->nlimb == pt->nlimb),
         "output may alias the plaintext only when the shapes match");
    prepare_out(out, ct->npoly, ct->nlimb);
    fhe::poly_mul_plain(*ct->c, out->data, ct->data, pt->data, ct->npoly, ct->nlimb);
  });
}

int fhe_add_plain(fhe_poly* out, const fhe_poly* ct, const fhe_poly* pt) {
  return guard([&] {
    same_ctx(ct, pt);
    same_ctx(out, ct);
    need(pt->npoly == 1 && pt->nlimb >= ct->nlimb, "plaintext must be one poly at >= limbs");
    // Reshaping the plaintext's own handle would free it before it is read.
    need(out != pt || (ct->npoly == 1 && ct->nlimb == pt->nlimb),
         "output may alias the plaintext only when the shapes match");
    prepare_out(out, ct->npoly, ct->nlimb);
    fhe::poly_add_plain(*ct->c, out->data, ct->data, pt->data, ct->npoly, ct->nlimb);
  });
}

int fhe_mul_const(fhe_poly* out, const fhe_poly* a, const uint64_t* cst) {
  return guard([&] {
    same_ctx(out, a);
    need(cst != nullptr, "null constants");
    prepare_out(out, a->npoly, a->nlimb);
    fhe::poly_mul_const(*a->c, out->data, a->data, cst, a->npoly, a->nlimb);
  });
}

int fhe_linear_wsum(fhe_poly* out, const fhe_poly* const* xs, const uint64_t* weights,
                    uint32_t count, uint32_t nlimb) {
  return guard([&] {
    need(out && xs && weights && count > 0, "null argument");
    fhe::Context& c = *out->c;
    need(nlimb >= 1 && nlimb <= c.L, "bad limb count");
    std::vector<const uint64_t*> ptrs(count);
    std::vector<uint32_t> nl(count);
    for (uint32_t i = 0; i < count; ++i) {
      need(xs[i] != nullptr, "null argument");
      same_ctx(out, xs[i]);
      need(xs[i] != out, "the output may not alias a term");
      need(xs[i]->npoly == 2 && xs[i]->nlimb >= nlimb, "terms are 2-poly ciphertexts with nlimb limbs");
    }
    prepare_out(out, 2, nlimb);
    for (uint32_t i = 0; i < count; ++i) {
      ptrs[i] = xs[i]->data;
      nl[i] = xs[i]->nlimb;
    }
    fhe::poly_linear_wsum(c, out->data, ptrs.data(), nl.data(), weights, count, nlimb);
  });
}

int fhe_add_const(fhe_poly* out, const fhe_poly* a, const uint64_t* cst) {
  return guard([&] {
    same_ctx(out, a);
    need(cst != nullptr, "null constants");
    prepare_out(out, a->npoly, a->nlimb);
    fhe::poly_add_const(*a->c, out->data, a->data, cst, a->npoly, a->nlimb);
  });
}

int fhe_mul_int(fhe_poly* out, const fhe_poly* a, int64_t v) {
  return guard([&] {
    same_ctx(out, a);
    std::vector<uint64_t> cst(a->nlimb);
    for (uint32_t j = 0; j < a->nlimb; ++j) {
      const uint64_t q = a->c->mods[j];
      const uint64_t r = (uint64_t)(v < 0 ? -(v + 1) : v) % q;
      cst[j] = v < 0 ? (q - 1 - r) : r;  // -(|v|) mod q without overflow
    }
    prepare_out(out, a->npoly, a->nlimb);
    fhe::poly_mul_const(*a->c, out->data, a->data, cst.data(), a->npoly, a->nlimb);
  });
}

int fhe_mod_raise(fhe_poly* out, const fhe_poly* a, uint32_t nlimb) {
  return guard([&] {
    same_ctx(out, a);
    need(a->nlimb >= 1 && a->npoly >= 1, "ModRaise needs at least one limb");
    need(nlimb >= 1 && nlimb <= a->c->L, "ModRaise output must have 1..L limbs");
    fhe::Context& c = *a->c;
    const uint32_t npoly = a->npoly, nl = a->nlimb;
    const uint64_t* src = a->data;
    write_result(out, a, npoly, nlimb, [&](uint64_t* dst) {
      fhe::poly_mod_raise(c, dst, nlimb, src, nl, npoly);
    });
  });
}

int fhe_rescale(fhe_poly* out, const fhe_poly* a) {
  return guard([&] {
    same_ctx(out, a);
    need(a->nlimb >= 2 && a->nlimb <= a->c->L, "rescale needs 2..L limbs");
    fhe::Context& c = *a->c;
    const uint32_t npoly = a->npoly, nq = a->nlimb;
    const uint64_t* src = a->data;
    write_result(out, a, npoly, nq - 1,
                 [&](uint64_t* dst) { fhe::poly_rescale(c, dst, src, npoly, nq); });
  });
}

int fhe_rescale_many(fhe_poly* const* outs, const fhe_poly* const* as, uint32_t count) {
  return guard([&] {
    need(outs && as, "null argument");
    if (count == 0) return;
    need(as[0] != nullptr, "null input");
    fhe::Context& c = *as[0]->c;
    const uint32_t npoly = as[0]->npoly, nq = as[0]->nlimb;
    need(nq >= 2 && nq <= c.L, "rescale needs 2..L limbs");
    for (uint32_t r = 0; r < count; ++r) {
      need(as[r] && outs[r], "null handle");
      same_ctx(outs[r], as[r]);
      need(as[r]->c == &c && as[r]->npoly == npoly && as[r]->nlimb == nq,
           "rescale_many needs inputs of one context and shape");
      for (uint32_t s = 0; s < r; ++s) need(outs[s] != outs[r], "outputs must be distinct");
    }
    for (uint32_t r = 0; r < count; ++r)
      for (uint32_t s = 0; s < count; ++s)
        need(outs[r] != as[s], "an output must not be one of the inputs");
    std::vector<uint64_t*> dst(count);
    std::vector<const uint64_t*> src(count);
    for (uint32_t r = 0; r < count; ++r) {
      prepare_out(outs[r], npoly, nq - 1);
      dst[r] = outs[r]->data;
      src[r] = as[r]->data;
    }
    fhe::poly_rescale_many(c, dst.data(), src.data(), count, npoly, nq);
  });
}

int fhe_tensor(fhe_poly* out3, const fhe_poly* a, const fhe_poly* b) {
  return guard([&] {
    same_ctx(a, b);
    same_ctx(out3, a);
    need(a->npoly == 2 && b->npoly == 2 && a->nlimb == b->nlimb, "tensor needs 2-poly cts");
    need(out3 != a && out3 != b, "tensor output must not alias an input");
    prepare_out(out3, 3, a->nlimb);
    fhe::poly_tensor(*a->c, out3->data, a->data, b->data, a->nlimb);
  });
}

int fhe_key_load(fhe_context* ctx, const uint64_t* host, fhe_key** out) {
  return guard([&] {
    need(ctx && host && out, "null argument");
    fhe::Context& c = *ctx->c;
    fhe_key* k = new_key(ctx->own);
    fhe::hip_check(hipMemcpyAsync(k->data, host, k->bytes, hipMemcpyHostToDevice, c.stream),
                   "key upload");
    fhe::key_to_montgomery(c, k->data);
    fhe::hip_check(hipStreamSynchronize(c.stream), "key sync");
    *out = k;
  });
}

int fhe_key_download(const fhe_key* k, uint64_t* host) {
  return guard([&] {
    need(k && host, "null argument");
    fhe::Context& c = *k->c;
    fhe::Scratch t(c, k->bytes / 8);
    fhe::key_from_montgomery(c, t.p, k->data);
    fhe::hip_check(hipMemcpyAsync(host, t.p, k->bytes, hipMemcpyDeviceToHost, c.stream),
                   "key download");
    fhe::hip_check(hipStreamSynchronize(c.stream), "key sync");
  });
}

int fhe_key_destroy(fhe_key* k) {
  return guard([&] {
    if (!k) return;
    k->c->release(k->data, k->bytes);
    delete k;
  });
}

static void check_key(const fhe_poly* p, const fhe_key* k) {
  need(p && k && p->c == k->c, "key belongs to another context");
}

int fhe_keyswitch(fhe_poly* out, const fhe_poly* a, const fhe_key* key) {
  return guard([&] {
    same_ctx(out, a);
    check_key(a, key);
    need(a->npoly == 1 && a->nlimb >= 1 && a->nlimb <= a->c->L, "keyswitch input is one poly");
    fhe::Context& c = *a->c;
    const uint32_t nq = a->nlimb;
    const uint64_t* src = a->data;
    write_result(out, a, 2, nq, [&](uint64_t* dst) {
      fhe::keyswitch(c, src, nq, key->data, fhe::KeySwitchOut{dst, nullptr, nullptr, 1});
    });
  });
}

int fhe_relinearize(fhe_poly* out, const fhe_poly* ct3, const fhe_key* key) {
  return guard([&] {
    same_ctx(out, ct3);
    check_key(ct3, key);
    need(ct3->npoly == 3 && ct3->nlimb <= ct3->c->L, "relinearize needs a 3-poly tensor");
    fhe::Context& c = *ct3->c;
    const uint32_t nq = ct3->nlimb;
    const size_t pl = (size_t)nq * c.n;
    const uint64_t* src = ct3->data;
    write_result(out, ct3, 2, nq, [&](uint64_t* dst) {
      fhe::keyswitch(c, src + 2 * pl, nq, key->data, fhe::KeySwitchOut{dst, src, src + pl, 1});
    });
  });
}

int fhe_relinearize_many(fhe_poly* const* outs, const fhe_poly* const* ct3s, uint32_t count,
                         const fhe_key* key) {
  return guard([&] {
    need(outs && ct3s, "null argument");
    if (count == 0) return;
    need(ct3s[0] != nullptr, "null tensor");
    fhe::Context& c = *ct3s[0]->c;
    const uint32_t nq = ct3s[0]->nlimb;
    for (uint32_t r = 0; r < count; ++r) {
      need(ct3s[r] && outs[r], "null handle");
      same_ctx(outs[r], ct3s[r]);
      need(ct3s[r]->c == &c && ct3s[r]->npoly == 3 && ct3s[r]->nlimb == nq && nq <= c.L,
           "relinearize_many needs 3-poly tensors of one context and level");
      check_key(ct3s[r], key);
      for (uint32_t s = 0; s < r; ++s) need(outs[s] != outs[r], "outputs must be distinct");
    }
    for (uint32_t r = 0; r < count; ++r)
      for (uint32_t s = 0; s < count; ++s)
        need(outs[r] != ct3s[s], "an output must not be one of the tensors");
    std::vector<uint64_t*> dst(count);
    std::vector<const uint64_t*> src(count);
    for (uint32_t r = 0; r < count; ++r) {
      prepare_out(outs[r], 2, nq);
      dst[r] = outs[r]->data;
      src[r] = ct3s[r]->data;
    }
    fhe::relinearize_many(c, dst.data(), src.data(), nq, key->data, count);
  });
}

int fhe_rotate(fhe_poly* out, const fhe_poly* ct, const fhe_key* key, uint32_t galois) {
  return guard([&] {
    same_ctx(out, ct);
    check_key(ct, key);
    need(ct->npoly == 2 && ct->nlimb <= ct->c->L, "rotate needs a 2-poly ciphertext");
    need((galois & 1) && galois < 2 * ct->c->n, "Galois element must be odd and < 2N");
    fhe::Context& c = *ct->c;
    const uint32_t nq = ct->nlimb;
    const uint64_t* src = ct->data;
    write_result(out, ct, 2, nq,
                 [&](uint64_t* dst) { fhe::rotate(c, dst, src, nq, key->data, galois); });
  });
}

// ---- rotation without allocation -------------------------------------------
// Device scratch of fhe_rotate_noalloc: one copy per GPU, held until the
// process ends.  In host code `scratch` names a host-side stand-in, never
// device memory: its device address comes from hipGetSymbolAddress, once per
// device, and only that address is handed to kernels.
constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
static __device__ __align__(256) uint64_t scratch[kNoAllocScratchBytes / 8];

namespace {
// One GPU's `scratch` and the ordering of the calls that use it.  A call
// holds `mu` while it binds the array and enqueues its work, and records
// `done` on its stream when it is enqueued; a call on another stream (a
// second context, or a caller stream) first makes its stream wait for
// `done`, so calls on one GPU never overlap on the array, whichever
// contexts and streams they come from.
struct ScratchDevice {
  uint64_t* ptr = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;  // stream `done` was last recorded on
  bool recorded = false;
  std::mutex mu;
};
std::mutex g_scratch_mu;
std::map<int, std::unique_ptr<ScratchDevice>> g_scratch;  // device -> its state

// Set-up, once per device with that device current: the array's device
// address and the ordering event.
ScratchDevice& scratch_for_device(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch.find(device);
  if (it != g_scratch.end()) return *it->second;
  int prev = 0;
  fhe::hip_check(hipGetDevice(&prev), "hipGetDevice");
  fhe::hip_check(hipSetDevice(device), "hipSetDevice");
  void* ptr = nullptr;
  hipEvent_t ev = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  fhe::hip_check(hipSetDevice(prev), "hipSetDevice");
  fhe::hip_check(e, "no-allocation scratch set-up");
  if (!ptr) throw fhe::HipError("hipGetSymbolAddress(scratch) returned no address");
  auto d = std::make_unique<ScratchDevice>();
  d->ptr = static_cast<uint64_t*>(ptr);
  d->done = ev;
  return *(g_scratch[device] = std::move(d));
}

// Orders one call after every earlier call on the same GPU (see
// ScratchDevice) and records its own completion when it leaves, also when
// it throws after enqueuing part of its work.
struct ScratchTurn {
  ScratchDevice& d;
  hipStream_t s;
  std::lock_guard<std::mutex> lk;
  ScratchTurn(ScratchDevice& dev, hipStream_t stream) : d(dev), s(stream), lk(dev.mu) {
    if (d.recorded && d.last != s)
      fhe::hip_check(hipStreamWaitEvent(s, d.done, 0), "no-allocation rotate: stream wait");
  }
  ~ScratchTurn() {
    if (hipEventRecord(d.done, s) == hipSuccess) {
      d.last = s;
      d.recorded = true;
    }
  }
};

// Scratch words a rotation at nq limbs takes from the arena: the ModUp
// digits, the ModUp input staging, the ModDown P limbs and y, and a
// ciphertext-sized result when the output aliases the input.  Each buffer
// is rounded up to 256 bytes as the arena does.
size_t rotate_scratch_words(const fhe::Context& c, uint32_t nq, bool aliased) {
  auto r = [](size_t w) { return (w + 31) & ~(size_t)31; };
  const size_t n = c.n, nd = fhe::num_digits(c, nq);
  size_t w = r(nd * (nq + c.K) * n) + r((size_t)nq * n) + r(2 * (size_t)c.K * n) +
             r(2 * (size_t)nq * n);
  if (aliased) w += r(2 * (size_t)nq * n);
  return w;
}

struct ArenaScope {
  fhe::Context& c;
  ArenaScope(fhe::Context& ctx, uint64_t* base, size_t words) : c(ctx) {
    c.arena.base = base;
    c.arena.words = words;
    c.arena.used = 0;
  }
  ~ArenaScope() {
    c.arena.base = nullptr;
    c.arena.words = c.arena.used = 0;
  }
};
}  // namespace

int fhe_rotate_noalloc(fhe_poly* out, const fhe_poly* ct, const fhe_key* key, uint32_t galois) {
  return guard([&] {
    same_ctx(out, ct);
    check_key(ct, key);
    need(ct->npoly == 2 && ct->nlimb >= 1 && ct->nlimb <= ct->c->L,
         "rotate needs a 2-poly ciphertext");
    need((galois & 1) && galois < 2 * ct->c->n, "Galois element must be odd and < 2N");
    fhe::Context& c = *ct->c;
    const uint32_t nq = ct->nlimb;
    need(out->npoly == 2 && out->nlimb == nq && out->data,
         "no-allocation rotate: the output must already hold 2 polys at the input's limbs");
    const bool aliased = out == ct;
    const size_t need_words = rotate_scratch_words(c, nq, aliased);
    if (need_words * 8 > kNoAllocScratchBytes)
      throw fhe::ArgError("no-allocation rotate: this shape needs " +
                          std::to_string(need_words * 8) + " bytes of scratch, above the " +
                          std::to_string(kNoAllocScratchBytes) + "-byte limit");
    if (!c.has_keyswitch_plans(nq))
      throw fhe::StateError(
          "no-allocation rotate: the conversion tables for this level are not built yet "
          "(any allocating key switch at this level builds them)");
    ScratchDevice& dev = scratch_for_device(c.device);
    ScratchTurn turn(dev, c.stream);
    ArenaScope arena(c, dev.ptr, kNoAllocScratchBytes / 8);
    if (!aliased) {
      fhe::rotate(c, out->data, ct->data, nq, key->data, galois);
      return;
    }
    fhe::Scratch t(c, 2 * (size_t)nq * c.n);
    fhe::rotate(c, t.p, ct->data, nq, key->data, galois);
    fhe::hip_check(hipMemcpyAsync(out->data, t.p, out->bytes, hipMemcpyDeviceToDevice, c.stream),
                   "rotate");
  });
}

int fhe_rotation_precompute(const fhe_poly* ct, fhe_poly** digits) {
  return guard([&] {
    need(ct && digits, "null argument");
    need(ct->npoly == 2 && ct->nlimb <= ct->c->L, "precompute needs a 2-poly ciphertext");
    fhe::Context& c = *ct->c;
    const uint32_t nq = ct->nlimb, nd = fhe::num_digits(c, nq);
    fhe_poly* d = new fhe_poly{ct->own, &c, 0, 0, nullptr, 0};
    try {
      reshape(d, nd, nq + c.K);
      fhe::modup(c, ct->data + (size_t)nq * c.n, nq, d->data);
    } catch (...) {
      fhe_poly_destroy(d);
      throw;
    }
    *digits = d;
  });
}

int fhe_rotate_hoisted(const fhe_poly* ct, const fhe_poly* digits, const fhe_key* const* keys,
                       const uint32_t* galois, uint32_t count, fhe_poly* const* outs) {
  return guard([&] {
    need(ct && digits && keys && galois && outs, "null argument");
    same_ctx(ct, digits);
    fhe::Context& c = *ct->c;
    const uint32_t nq = ct->nlimb, ne = nq + c.K;
    need(ct->npoly == 2 && digits->npoly == fhe::num_digits(c, nq) && digits->nlimb == ne,
         "digits do not belong to this ciphertext level");
    for (uint32_t r = 0; r < count; ++r) {
      check_key(ct, keys[r]);
      need(outs[r] && outs[r]->c == &c && outs[r] != ct && outs[r] != digits,
           "bad output handle");
      need((galois[r] & 1) && galois[r] < 2 * c.n, "Galois element must be odd and < 2N");
      for (uint32_t s = 0; s < r; ++s) need(outs[s] != outs[r], "outputs must be distinct");
    }
    for (uint32_t r = 0; r < count; ++r) prepare_out(outs[r], 2, nq);
    std::vector<const uint64_t*> kp(count);
    std::vector<fhe::KeySwitchOut> ko(count);
    for (uint32_t r = 0; r < count; ++r) {
      kp[r] = keys[r]->data;
      ko[r] = fhe::KeySwitchOut{outs[r]->data, ct->data, nullptr, galois[r]};
    }
    fhe::keyswitch_hoisted(c, digits->data, nq, kp.data(), ko.data(), count);
  });
}

int fhe_rotate_many(fhe_poly* const* outs, const fhe_poly* const* cts, const fhe_key* const* keys,
                    const uint32_t* galois, uint32_t count) {
  return guard([&] {
    need(outs && cts && keys && galois, "null argument");
    if (count == 0) return;
    need(cts[0] != nullptr, "null ciphertext");
    fhe::Context& c = *cts[0]->c;
    const uint32_t nq = cts[0]->nlimb;
    for (uint32_t r = 0; r < count; ++r) {
      need(cts[r] && outs[r], "null handle");
      same_ctx(outs[r], cts[r]);
      need(cts[r]->c == &c && cts[r]->npoly == 2 && cts[r]->nlimb == nq && nq <= c.L,
           "rotate_many needs 2-poly ciphertexts of one context and level");
      check_key(cts[r], keys[r]);
      need((galois[r] & 1) && galois[r] < 2 * c.n, "Galois element must be odd and < 2N");
      for (uint32_t s = 0; s < r; ++s) need(outs[s] != outs[r], "outputs must be distinct");
    }
    // Outputs that alias an input are written to scratch and copied after.
    const size_t pl = 2 * (size_t)nq * c.n;
    std::vector<uint8_t> alias(count, 0);
    uint32_t naliased = 0;
    for (uint32_t r = 0; r < count; ++r)
      for (uint32_t s = 0; s < count; ++s)
        if (outs[r] == cts[s]) alias[r] = 1;
    for (uint32_t r = 0; r < count; ++r) naliased += alias[r];
    fhe::Scratch tmp(c, std::max<size_t>(1, naliased * pl));
    std::vector<uint64_t*> dst(count);
    std::vector<const uint64_t*> src(count), kp(count);
    for (uint32_t r = 0, t = 0; r < count; ++r) {
      if (!alias[r]) prepare_out(outs[r], 2, nq);
      dst[r] = alias[r] ? tmp.p + (t++) * pl : outs[r]->data;
      src[r] = cts[r]->data;
      kp[r] = keys[r]->data;
    }
    fhe::rotate_many(c, dst.data(), src.data(), nq, kp.data(), galois, count);
    for (uint32_t r = 0; r < count; ++r) {
      if (!alias[r]) continue;  // an input handle: already [2][nq]
      fhe::hip_check(hipMemcpyAsync(outs[r]->data, dst[r], pl * 8, hipMemcpyDeviceToDevice,
                                    c.stream),
                     "rotate_many");
    }
  });
}

static void linear_transform_checked(fhe_poly* const* outs, const fhe_poly* const* cts,
                                     uint32_t ncts, const fhe_poly* const* pts, uint32_t count,
                                     uint32_t bstep, const fhe_key* const* baby_keys,
                                     const uint32_t* baby_galois, const fhe_key* const* giant_keys,
                                     const uint32_t* giant_galois, uint32_t n_giant_keys) {
  need(outs && cts && pts, "null argument");
  need(ncts >= 1 && ncts <= 64, "1..64 ciphertexts per linear transform call");
  const fhe_poly* ct = cts[0];
  need(ct != nullptr, "null argument");
  fhe::Context& c = *ct->c;
  const uint32_t nq = ct->nlimb;
  for (uint32_t i = 0; i < ncts; ++i) {
    need(cts[i] && outs[i], "null argument");
    same_ctx(outs[i], cts[i]);
    need(cts[i]->c == &c, "ciphertexts belong to different contexts");
    need(cts[i]->npoly == 2 && cts[i]->nlimb <= c.L,
         "linear transform needs a 2-poly ciphertext");
    need(cts[i]->nlimb == nq, "ciphertexts of one call must share their limb count");
    for (uint32_t j = 0; j < i; ++j) need(outs[j] != outs[i], "outputs must be distinct");
  }
  need(count >= 1 && bstep >= 1 && bstep <= fhe::MAC_TABLE,
       "need count >= 1 and 1 <= bstep <= 64");
  const uint32_t giants = (count + bstep - 1) / bstep;
  std::vector<const uint64_t*> pp(count, nullptr);
  bool any = false;
  for (uint32_t k = 0; k < count; ++k) {
    if (!pts[k]) continue;
    need(pts[k]->c == &c && pts[k]->npoly == 1 && pts[k]->nlimb >= nq,
         "diagonal must be a one-poly plaintext with at least the ciphertext's limbs");
    // Shaping an output as a ciphertext would free this diagonal's storage
    // while the transform still reads it.
    for (uint32_t i = 0; i < ncts; ++i)
      need(pts[k] != outs[i], "the output must not be one of the diagonals");
    pp[k] = pts[k]->data;
    any = true;
  }
  need(any, "linear transform has no nonzero diagonal");
  const uint32_t nb = std::min(bstep, count);
  std::vector<const uint64_t*> bk(nb, nullptr);
  std::vector<uint32_t> bg(nb, 1);
  for (uint32_t b = 0; b < nb; ++b) {
    if (!baby_keys || !baby_keys[b]) continue;
    need(baby_galois != nullptr, "null argument");
    check_key(ct, baby_keys[b]);
    need((baby_galois[b] & 1) && baby_galois[b] < 2 * c.n, "bad Galois element");
    bk[b] = baby_keys[b]->data;
    bg[b] = baby_galois[b];
  }
  std::vector<const uint64_t*> gk;
  std::vector<uint32_t> gg;
  if (giants > 1) {
    need(n_giant_keys == 1 || n_giant_keys == giants - 1,
         "one giant-step key, or one per giant step");
    need(giant_keys && giant_galois, "giant-step key required when count > bstep");
    for (uint32_t g = 0; g < n_giant_keys; ++g) {
      need(giant_keys[g] != nullptr, "giant-step key required when count > bstep");
      check_key(ct, giant_keys[g]);
      need((giant_galois[g] & 1) && giant_galois[g] < 2 * c.n, "bad Galois element");
      gk.push_back(giant_keys[g]->data);
      gg.push_back(giant_galois[g]);
    }
  }
  // An output that is some input keeps its storage (same shape); every
  // input is read before any output is written.
  std::vector<const uint64_t*> src(ncts);
  for (uint32_t i = 0; i < ncts; ++i) src[i] = cts[i]->data;
  std::vector<uint64_t*> dst(ncts);
  for (uint32_t i = 0; i < ncts; ++i) {
    prepare_out(outs[i], 2, nq);
    dst[i] = outs[i]->data;
  }
  fhe::linear_transform_many(c, dst.data(), src.data(), ncts, nq, pp.data(), count, bstep,
                             bk.data(), bg.data(), gk.data(), gg.data(),
                             giants > 1 ? n_giant_keys : 0);
}

int fhe_linear_transform(fhe_poly* out, const fhe_poly* ct, const fhe_poly* const* pts,
                         uint32_t count, uint32_t bstep, const fhe_key* const* baby_keys,
                         const uint32_t* baby_galois, const fhe_key* giant_key,
                         uint32_t giant_galois) {
  return guard([&] {
    need(bstep <= 1 || (baby_keys && baby_galois), "null argument");
    const uint32_t nb = std::min(bstep, count);
    // baby b >= 1 of the hoisted form is baby_keys[b - 1] here; baby 0 is ct
    std::vector<const fhe_key*> bk(std::max<uint32_t>(nb, 1), nullptr);
    std::vector<uint32_t> bg(std::max<uint32_t>(nb, 1), 1);
    for (uint32_t b = 1; b < nb; ++b) {
      bk[b] = baby_keys[b - 1];
      bg[b] = baby_galois[b - 1];
    }
    need(out && ct, "null argument");
    linear_transform_checked(&out, &ct, 1, pts, count, bstep, bk.data(), bg.data(), &giant_key,
                             &giant_galois, 1);
  });
}

int fhe_linear_transform_hoisted(fhe_poly* out, const fhe_poly* ct, const fhe_poly* const* pts,
                                 uint32_t count, uint32_t bstep, const fhe_key* const* baby_keys,
                                 const uint32_t* baby_galois, const fhe_key* const* giant_keys,
                                 const uint32_t* giant_galois, uint32_t n_giant_keys) {
  return guard([&] {
    need(baby_keys && baby_galois && out && ct, "null argument");
    linear_transform_checked(&out, &ct, 1, pts, count, bstep, baby_keys, baby_galois, giant_keys,
                             giant_galois, n_giant_keys);
  });
}

int fhe_linear_transform_hoisted_many(fhe_poly* const* outs, const fhe_poly* const* cts,
                                      uint32_t ncts, const fhe_poly* const* pts, uint32_t count,
                                      uint32_t bstep, const fhe_key* const* baby_keys,
                                      const uint32_t* baby_galois,
                                      const fhe_key* const* giant_keys,
                                      const uint32_t* giant_galois, uint32_t n_giant_keys) {
  return guard([&] {
    need(baby_keys && baby_galois, "null argument");
    linear_transform_checked(outs, cts, ncts, pts, count, bstep, baby_keys, baby_galois,
                             giant_keys, giant_galois, n_giant_keys);
  });
}

int fhe_encode(fhe_context* ctx, const double* re, const double* im, uint32_t count,
               uint32_t slots, double scale, uint32_t nlimb, fhe_poly* out) {
  return guard([&] {
    need(ctx && out && out->c == ctx->c && (re || count == 0), "null argument");
    fhe::Context& c = *ctx->c;
    prepare_out(out, 1, nlimb);
    if (!fhe::encode(c, re, im, count, slots, scale, nlimb, out->data))
      throw std::out_of_range("encode: a scaled coefficient does not fit in 62 bits");
  });
}

int fhe_encode_many(fhe_context* ctx, const double* re, const double* im, uint32_t count,
                    uint32_t nvec, uint32_t slots, double scale, uint32_t nlimb,
                    fhe_poly* const* outs) {
  return guard([&] {
    need(ctx && (outs || nvec == 0) && (re || count == 0 || nvec == 0), "null argument");
    fhe::Context& c = *ctx->c;
    std::vector<uint64_t*> ptrs(nvec);
    std::vector<const fhe_poly*> seen(outs, outs + nvec);
    for (const fhe_poly* o : seen) need(o && o->c == ctx->c, "null argument");
    std::sort(seen.begin(), seen.end());
    need(std::adjacent_find(seen.begin(), seen.end()) == seen.end(), "an output appears twice");
    for (uint32_t r = 0; r < nvec; ++r) {
      prepare_out(outs[r], 1, nlimb);
      ptrs[r] = outs[r]->data;
    }
    if (!fhe::encode_many(c, re, im, count, nvec, slots, scale, nlimb, ptrs.data()))
      throw std::out_of_range("encode: a scaled coefficient does not fit in 62 bits");
  });
}

int fhe_decode(fhe_context* ctx, const fhe_poly* pt, uint32_t slots, double scale, double* re,
               double* im) {
  return guard([&] {
    need(ctx && pt && re && pt->c == ctx->c, "null argument");
    need(pt->npoly == 1, "decode takes a one-poly plaintext");
    fhe::decode(*ctx->c, pt->data, pt->nlimb, slots, scale, re, im);
  });
}

int fhe_context_set_sampling(fhe_context* ctx, int mode, const uint8_t* key32) {
  return guard([&] {
    need(ctx != nullptr, "null argument");
    fhe::SamplingKey k;
    if (mode == FHE_SAMPLING_CHACHA20) {
      if (key32) {
        for (int i = 0; i < 8; ++i)
          k.master[i] = (uint32_t)key32[4 * i] | ((uint32_t)key32[4 * i + 1] << 8) |
                        ((uint32_t)key32[4 * i + 2] << 16) | ((uint32_t)key32[4 * i + 3] << 24);
      } else {
        fhe::fill_entropy(k.master, sizeof(k.master));
      }
      k.secure = true;
    } else {
      need(mode == FHE_SAMPLING_SEEDED, "sampling mode must be FHE_SAMPLING_CHACHA20 or "
                                        "FHE_SAMPLING_SEEDED");
      need(key32 == nullptr, "the seeded sampling family takes no key");
      k.secure = false;
    }
    ctx->c->sampling = k;
  });
}

int fhe_keygen_secret(fhe_context* ctx, uint64_t seed, int64_t* s_coef) {
  return guard([&] {
    need(ctx && s_coef, "null argument");
    fhe::sample_secret_host(*ctx->c, seed, s_coef);
  });
}

int fhe_keygen_secret_sparse(fhe_context* ctx, uint64_t seed, uint32_t h, int64_t* s_coef) {
  return guard([&] {
    need(ctx && s_coef, "null argument");
    need(h >= 1 && h <= ctx->c->n, "sparse secret: Hamming weight must be in [1, N]");
    fhe::sample_sparse_secret_host(*ctx->c, seed, s_coef, h);
  });
}

int fhe_keygen_public(fhe_context* ctx, const int64_t* s_coef, uint64_t seed, fhe_poly* pk) {
  return guard([&] {
    need(ctx && s_coef && pk && pk->c == ctx->c, "null argument");
    prepare_out(pk, 2, ctx->c->L);
    fhe::keygen_public(*ctx->c, s_coef, seed, pk->data);
  });
}

int fhe_keygen_relin(fhe_context* ctx, const int64_t* s_coef, uint64_t seed, fhe_key** out) {
  return guard([&] {
    need(ctx && s_coef && out, "null argument");
    fhe::Context& c = *ctx->c;
    fhe_key* k = new_key(ctx->own);
    try {
      fhe::keygen_relin(c, s_coef, seed, k->data);
      fhe::key_to_montgomery(c, k->data);
      fhe::hip_check(hipStreamSynchronize(c.stream), "keygen");
    } catch (...) {
      fhe_key_destroy(k);
      throw;
    }
    *out = k;
  });
}

int fhe_keygen_galois(fhe_context* ctx, const int64_t* s_coef, uint32_t galois, uint64_t seed,
                      fhe_key** out) {
  return guard([&] {
    need(ctx && s_coef && out, "null argument");
    fhe::Context& c = *ctx->c;
    need((galois & 1) && galois < 2 * c.n, "Galois element must be odd and < 2N");
    fhe_key* k = new_key(ctx->own);
    try {
      fhe::keygen_galois(c, s_coef, galois, seed, k->data);
      fhe::key_to_montgomery(c, k->data);
      fhe::hip_check(hipStreamSynchronize(c.stream), "keygen");
    } catch (...) {
      fhe_key_destroy(k);
      throw;
    }
    *out = k;
  });
}

int fhe_encrypt(fhe_poly* ct, const fhe_poly* pk, const fhe_poly* pt, uint64_t seed) {
  return guard([&] {
    same_ctx(pk, pt);
    same_ctx(ct, pk);
    need(pk->npoly == 2 && pt->npoly == 1 && pt->nlimb <= pk->nlimb, "bad key or plaintext");
    need(ct != pt && ct != pk, "ciphertext must not alias an input");
    prepare_out(ct, 2, pt->nlimb);
    fhe::encrypt_pk(*pt->c, pk->data, pt->data, pt->nlimb, seed, ct->data);
  });
}

int fhe_decrypt(fhe_poly* pt, const fhe_poly* ct, const int64_t* s_coef) {
  return guard([&] {
    same_ctx(pt, ct);
    need(s_coef != nullptr && ct->npoly >= 2 && ct->npoly <= 3, "bad ciphertext");
    need(pt != ct, "plaintext must not alias the ciphertext");
    prepare_out(pt, 1, ct->nlimb);
    fhe::decrypt(*ct->c, ct->data, ct->npoly, ct->nlimb, s_coef, pt->data);
  });
}

}  // extern "C"
