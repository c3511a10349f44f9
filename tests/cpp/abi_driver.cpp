// abi_driver.cpp -- the C++ twin of the Rust `hip` module (integration/rust/src/gpu/hip.rs): loads
// libapeiron_hip.so with dlopen, resolves the same entry points by name, maps every status to the
// one error value the Rust module maps it to, and runs the host-form projection calls.  Built by
// apeiron_amd/build.py with g++ (no HIP headers or libraries: only include/apeiron_hip.h for the
// constants); driven by tests/test_cpp_driver.py (CPU) and tests/test_gpu_cpp_driver.py (GPU).
//
// Usage:
//   abi_driver LIB status            the status -> error table, one line per code 0..26
//   abi_driver LIB probe             load, resolve, ah_init(0): "DEVICE ok" or "SKIP <reason>"
//   abi_driver LIB run IN OUT        one case file through upload / matvec / matmat / quant_act
//   abi_driver LIB engine IN OUT     the device-resident forms (see run_engine)
//
// Case file (little-endian): u32 ggml_type, u64 n_out, u64 n_in, u64 n_tok, u64 raw_len, raw bytes,
// codes [n_tok][n_in] i8, scales [n_tok][ceil(n_in/32)] i64, x [n_in] i64 (a Q32.32 activation for
// quant_act).  Output file: i32 upload status, i32 matvec status, f32 y0 [n_out], i32 matmat status,
// f32 Y [n_tok][n_out], i32 quant status, i8 codes [n_in], i64 scales [ceil(n_in/32)], u32 refusal
// bits (ah_last_refusal_bits after the upload).
#include "apeiron_hip.h"

#include <dlfcn.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

using Init = int32_t (*)(int32_t, ah_ctx **);
using Destroy = int32_t (*)(ah_ctx *);
using StatusStr = const char *(*)(int32_t);
using Upload = int32_t (*)(ah_ctx *, uint32_t, const void *, size_t, size_t, size_t, ah_tensor **);
using FreeTensor = int32_t (*)(ah_ctx *, ah_tensor *);
using MatvecQ8 = int32_t (*)(ah_ctx *, const ah_tensor *, const int8_t *, const int64_t *, size_t, float *);
using MatmatQ8 = int32_t (*)(ah_ctx *, const ah_tensor *, const int8_t *, const int64_t *, size_t, float *);
using QuantAct = int32_t (*)(ah_ctx *, const int64_t *, size_t, int8_t *, int64_t *);
using RefusalBits = int32_t (*)(const ah_ctx *, uint32_t *);
using ProbeMfma = int32_t (*)(ah_ctx *, uint32_t, double *);
using SyncStatus = int32_t (*)(ah_ctx *, void *);
using GemvQ8Dev = int32_t (*)(ah_ctx *, const ah_tensor *, const int8_t *, const int64_t *, float *, void *);
using GemmGroupQ8Dev = int32_t (*)(ah_ctx *, size_t, const ah_tensor *const *, const int8_t *, const int64_t *,
                                   size_t, float *const *, void *);
using FfnQ8Dev = int32_t (*)(ah_ctx *, const ah_tensor *, const ah_tensor *, const ah_tensor *, const int8_t *,
                             const int64_t *, float *, int8_t *, int64_t *, void *);
using FfnPrefillQ8Dev = int32_t (*)(ah_ctx *, const ah_tensor *, const ah_tensor *, const ah_tensor *,
                                    const int8_t *, const int64_t *, size_t, float *, int8_t *, int64_t *, void *);
using DevAlloc = int32_t (*)(ah_ctx *, size_t, void **);
using DevFree = int32_t (*)(ah_ctx *, void *);
using Copy = int32_t (*)(ah_ctx *, void *, const void *, size_t, void *);

struct Fns {
    Init init;
    Destroy destroy;
    StatusStr status_str;
    Upload upload;
    FreeTensor free_tensor;
    MatvecQ8 matvec;
    MatmatQ8 matmat;
    QuantAct quant;
    RefusalBits refusal_bits;
    ProbeMfma probe;
    SyncStatus sync;
    GemvQ8Dev gemv_q8;
    GemmGroupQ8Dev gemm_group_q8;
    FfnQ8Dev ffn_q8;
    FfnPrefillQ8Dev ffn_prefill_q8;
    DevAlloc dev_alloc;
    DevFree dev_free;
    Copy to_dev;
    Copy to_host;
};

template <typename T>
bool sym(void *lib, const char *name, T &out) {
    void *p = dlsym(lib, name);
    if (!p) {
        std::printf("SKIP missing symbol %s\n", name);
        return false;
    }
    static_assert(sizeof(T) == sizeof(void *), "function pointers are pointer-sized");
    std::memcpy(&out, &p, sizeof(p));
    return true;
}

bool resolve(void *lib, Fns &f) {
    return sym(lib, "ah_init", f.init) && sym(lib, "ah_destroy", f.destroy) &&
           sym(lib, "ah_status_str", f.status_str) && sym(lib, "ah_upload_weight", f.upload) &&
           sym(lib, "ah_free_tensor", f.free_tensor) && sym(lib, "ah_matvec_q8act", f.matvec) &&
           sym(lib, "ah_matmat_q8act", f.matmat) && sym(lib, "ah_quant_act", f.quant) &&
           sym(lib, "ah_last_refusal_bits", f.refusal_bits) && sym(lib, "ah_probe_mfma_peak", f.probe) &&
           sym(lib, "ah_sync_status", f.sync) && sym(lib, "ah_gemv_q8_dev", f.gemv_q8) &&
           sym(lib, "ah_gemm_group_q8_dev", f.gemm_group_q8) && sym(lib, "ah_ffn_q8_dev", f.ffn_q8) &&
           sym(lib, "ah_ffn_prefill_q8_dev", f.ffn_prefill_q8) && sym(lib, "ah_dev_alloc", f.dev_alloc) &&
           sym(lib, "ah_dev_free", f.dev_free) && sym(lib, "ah_copy_to_dev", f.to_dev) &&
           sym(lib, "ah_copy_to_host", f.to_host);
}

// The error value HipError::from_status gives each status (the Rust module's mapping, by name).
const char *rust_error(int32_t st) {
    switch (st) {
    case AH_OK: return "Ok";
    case AH_ERR_SHAPE_MISMATCH: return "Matvec(ShapeMismatch)";
    case AH_ERR_ROW_LENGTH: return "Matvec(RowLength)";
    case AH_ERR_SHORT_PAYLOAD: return "Matvec(ShortPayload)";
    case AH_ERR_LENGTH_OVERFLOW: return "Matvec(LengthOverflow)";
    case AH_ERR_UNSUPPORTED_QUANT: return "Matvec(UnsupportedQuant)";
    case AH_ERR_NONFINITE_SCALE: return "Matvec(Dequant(NonFiniteScale))";
    case AH_ERR_FIXED_OVERFLOW: return "Matvec(Dequant(FixedOverflow))";
    case AH_ERR_ACCUMULATOR_OVERFLOW: return "Matvec(AccumulatorOverflow)";
    case AH_ERR_OUTPUT_OVERFLOW: return "Matvec(OutputOverflow)";
    case AH_ERR_NONFINITE_INPUT: return "Input(NonFinite)";
    case AH_ERR_INPUT_RANGE: return "Input(OutOfRange)";
    case AH_ERR_FFN_OVERFLOW: return "Ffn(Overflow)";
    case AH_ERR_EXP_RANGE: return "Ffn(ExpOutOfRange)";
    case AH_ERR_ZERO_DENOMINATOR: return "Ffn(ZeroDenominator)";
    default: return "Backend";
    }
}

struct Reader {
    std::vector<uint8_t> b;
    size_t at = 0;
    bool ok = true;
    template <typename T> T get() {
        T v{};
        if (at + sizeof(T) > b.size()) {
            ok = false;
            return v;
        }
        std::memcpy(&v, b.data() + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    template <typename T> std::vector<T> arr(size_t n) {
        std::vector<T> v(n);
        if (at + n * sizeof(T) > b.size()) {
            ok = false;
            return v;
        }
        if (n) std::memcpy(v.data(), b.data() + at, n * sizeof(T));
        at += n * sizeof(T);
        return v;
    }
};

template <typename T> void put(std::FILE *f, const T &v) { std::fwrite(&v, sizeof(T), 1, f); }
template <typename T> void put_arr(std::FILE *f, const std::vector<T> &v) {
    if (!v.empty()) std::fwrite(v.data(), sizeof(T), v.size(), f);
}

int run_case(const Fns &f, ah_ctx *ctx, const char *in_path, const char *out_path) {
    Reader r;
    {
        std::FILE *fi = std::fopen(in_path, "rb");
        if (!fi) return 2;
        std::fseek(fi, 0, SEEK_END);
        r.b.resize((size_t)std::ftell(fi));
        std::fseek(fi, 0, SEEK_SET);
        const size_t got = r.b.empty() ? 0 : std::fread(r.b.data(), 1, r.b.size(), fi);
        std::fclose(fi);
        if (got != r.b.size()) return 2;
    }
    const uint32_t type = r.get<uint32_t>();
    const uint64_t n_out = r.get<uint64_t>(), n_in = r.get<uint64_t>(), n_tok = r.get<uint64_t>();
    const uint64_t raw_len = r.get<uint64_t>();
    const size_t nb = (size_t)((n_in + 31) / 32);
    const std::vector<uint8_t> raw = r.arr<uint8_t>(raw_len);
    const std::vector<int8_t> codes = r.arr<int8_t>(n_tok * n_in);
    const std::vector<int64_t> scales = r.arr<int64_t>(n_tok * nb);
    const std::vector<int64_t> x = r.arr<int64_t>(n_in);
    if (!r.ok || n_tok == 0) return 2;

    std::FILE *fo = std::fopen(out_path, "wb");
    if (!fo) return 2;
    ah_tensor *t = nullptr;
    const int32_t su = f.upload(ctx, type, raw.data(), raw.size(), n_out, n_in, &t);
    put(fo, su);
    uint32_t bits = 0;
    f.refusal_bits(ctx, &bits);
    std::vector<float> y0(n_out, 0.0f), Y(n_tok * n_out, 0.0f);
    int32_t sv = AH_ERR_INVALID_ARG, sm = AH_ERR_INVALID_ARG;
    if (su == AH_OK) {
        sv = f.matvec(ctx, t, codes.data(), scales.data(), n_in, y0.data());
        sm = f.matmat(ctx, t, codes.data(), scales.data(), n_tok, Y.data());
    }
    put(fo, sv);
    put_arr(fo, y0);
    put(fo, sm);
    put_arr(fo, Y);
    std::vector<int8_t> qc(n_in, 0);
    std::vector<int64_t> qs(nb, 0);
    const int32_t sq = f.quant(ctx, x.data(), n_in, qc.data(), qs.data());
    put(fo, sq);
    put_arr(fo, qc);
    put_arr(fo, qs);
    put(fo, bits);
    std::fclose(fo);
    if (t) f.free_tensor(ctx, t);
    std::printf("RUN upload %s, matvec %s, matmat %s, quant_act %s\n", rust_error(su), rust_error(sv),
                rust_error(sm), rust_error(sq));
    return 0;
}

// The device-resident forms in the order the Rust module's Hip methods make them
// (projections_q8act, ffn_q8act, matmat_group_q8act, ffn_cols_q8act): one staging region carved
// into 256-byte pieces, one upload of the QuantAct per call, the call's launches, one
// ah_sync_status, the outputs downloaded.
//
// Case file: u32 gate/up type, u32 down type, u64 n_embd, u64 n_ff, u64 n_tok, then three
// payloads (u64 length + bytes: gate, up, down), codes [n_tok][n_embd] i8, scales
// [n_tok][ceil(n_embd/32)] i64.  Output file: i32 upload statuses x3; i32 projections status,
// f32 gate [n_ff], f32 up [n_ff] (token 0); i32 ffn status, f32 y [n_embd], i8 hidden codes
// [n_ff], i64 hidden scales [ceil(n_ff/32)] (token 0); i32 group status, f32 gate [n_tok][n_ff],
// f32 up [n_tok][n_ff]; i32 column-FFN status, f32 y [n_tok][n_embd], i8 hidden codes
// [n_tok][n_ff], i64 hidden scales [n_tok][ceil(n_ff/32)].
size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

int run_engine(const Fns &f, ah_ctx *ctx, const char *in_path, const char *out_path) {
    Reader r;
    {
        std::FILE *fi = std::fopen(in_path, "rb");
        if (!fi) return 2;
        std::fseek(fi, 0, SEEK_END);
        r.b.resize((size_t)std::ftell(fi));
        std::fseek(fi, 0, SEEK_SET);
        const size_t got = r.b.empty() ? 0 : std::fread(r.b.data(), 1, r.b.size(), fi);
        std::fclose(fi);
        if (got != r.b.size()) return 2;
    }
    const uint32_t gt = r.get<uint32_t>(), dt = r.get<uint32_t>();
    const uint64_t n_embd = r.get<uint64_t>(), n_ff = r.get<uint64_t>(), n_tok = r.get<uint64_t>();
    std::vector<uint8_t> raw[3];
    for (auto &w : raw) w = r.arr<uint8_t>(r.get<uint64_t>());
    const size_t nb = (size_t)((n_embd + 31) / 32), nbh = (size_t)((n_ff + 31) / 32);
    const std::vector<int8_t> codes = r.arr<int8_t>(n_tok * n_embd);
    const std::vector<int64_t> scales = r.arr<int64_t>(n_tok * nb);
    if (!r.ok || n_tok == 0) return 2;
    std::FILE *fo = std::fopen(out_path, "wb");
    if (!fo) return 2;
    ah_tensor *t[3] = {nullptr, nullptr, nullptr};
    const uint32_t types[3] = {gt, gt, dt};
    const size_t shape[3][2] = {{n_ff, n_embd}, {n_ff, n_embd}, {n_embd, n_ff}};
    int32_t su[3];
    for (int i = 0; i < 3; ++i) {
        su[i] = f.upload(ctx, types[i], raw[i].data(), raw[i].size(), shape[i][0], shape[i][1], &t[i]);
        put(fo, su[i]);
    }
    if (su[0] || su[1] || su[2]) {
        std::fclose(fo);
        std::printf("ENGINE upload refused\n");
        return 0;
    }
    // the staging region, sized for the largest call (the column FFN)
    const size_t pieces[5] = {a256(n_tok * n_embd), a256(8 * n_tok * nb), a256(4 * n_tok * n_embd),
                              a256(n_tok * n_ff), a256(8 * n_tok * nbh)};
    const size_t out_g = a256(4 * n_tok * n_ff);
    size_t total = pieces[0] + pieces[1] + 2 * out_g;
    const size_t ffn_total = pieces[0] + pieces[1] + pieces[2] + pieces[3] + pieces[4];
    total = total > ffn_total ? total : ffn_total;
    void *stage = nullptr;
    if (f.dev_alloc(ctx, total, &stage) != AH_OK) {
        std::fclose(fo);
        return 3;
    }
    uint8_t *B = static_cast<uint8_t *>(stage);
    int8_t *d_codes = reinterpret_cast<int8_t *>(B);
    int64_t *d_scales = reinterpret_cast<int64_t *>(B + pieces[0]);
    uint8_t *o = B + pieces[0] + pieces[1];
    int32_t st;
    // projections_q8act: token 0 through gate and up
    std::vector<float> yg(n_ff), yu(n_ff);
    st = f.to_dev(ctx, d_codes, codes.data(), n_embd, nullptr);
    if (!st) st = f.to_dev(ctx, d_scales, scales.data(), 8 * nb, nullptr);
    float *dg = reinterpret_cast<float *>(o), *du = reinterpret_cast<float *>(o + out_g);
    if (!st) st = f.gemv_q8(ctx, t[0], d_codes, d_scales, dg, nullptr);
    if (!st) st = f.gemv_q8(ctx, t[1], d_codes, d_scales, du, nullptr);
    if (!st) st = f.sync(ctx, nullptr);
    const int32_t sp = st;
    if (!st) st = f.to_host(ctx, yg.data(), dg, 4 * n_ff, nullptr);
    if (!st) st = f.to_host(ctx, yu.data(), du, 4 * n_ff, nullptr);
    put(fo, sp);
    put_arr(fo, yg);
    put_arr(fo, yu);
    // ffn_q8act: token 0 through the FFN (hidden QuantAct kept on the device, read back here to check)
    std::vector<float> y(n_embd);
    std::vector<int8_t> hc(n_ff);
    std::vector<int64_t> hs(nbh);
    float *dy = reinterpret_cast<float *>(B + pieces[0] + pieces[1]);
    int8_t *dhc = reinterpret_cast<int8_t *>(B + pieces[0] + pieces[1] + pieces[2]);
    int64_t *dhs = reinterpret_cast<int64_t *>(B + pieces[0] + pieces[1] + pieces[2] + pieces[3]);
    st = f.ffn_q8(ctx, t[0], t[1], t[2], d_codes, d_scales, dy, dhc, dhs, nullptr);
    if (!st) st = f.sync(ctx, nullptr);
    const int32_t sf = st;
    if (!st) st = f.to_host(ctx, y.data(), dy, 4 * n_embd, nullptr);
    if (!st) st = f.to_host(ctx, hc.data(), dhc, n_ff, nullptr);
    if (!st) st = f.to_host(ctx, hs.data(), dhs, 8 * nbh, nullptr);
    put(fo, sf);
    put_arr(fo, y);
    put_arr(fo, hc);
    put_arr(fo, hs);
    // matmat_group_q8act: every column through gate and up as one group
    std::vector<float> Yg(n_tok * n_ff), Yu(n_tok * n_ff);
    st = f.to_dev(ctx, d_codes, codes.data(), n_tok * n_embd, nullptr);
    if (!st) st = f.to_dev(ctx, d_scales, scales.data(), 8 * n_tok * nb, nullptr);
    const ah_tensor *gu[2] = {t[0], t[1]};
    float *const ys[2] = {dg, du};
    if (!st) st = f.gemm_group_q8(ctx, 2, gu, d_codes, d_scales, n_tok, ys, nullptr);
    if (!st) st = f.sync(ctx, nullptr);
    const int32_t sg = st;
    if (!st) st = f.to_host(ctx, Yg.data(), dg, 4 * n_tok * n_ff, nullptr);
    if (!st) st = f.to_host(ctx, Yu.data(), du, 4 * n_tok * n_ff, nullptr);
    put(fo, sg);
    put_arr(fo, Yg);
    put_arr(fo, Yu);
    // ffn_cols_q8act: every column through the FFN
    std::vector<float> Y(n_tok * n_embd);
    std::vector<int8_t> HC(n_tok * n_ff);
    std::vector<int64_t> HS(n_tok * nbh);
    st = f.ffn_prefill_q8(ctx, t[0], t[1], t[2], d_codes, d_scales, n_tok, dy, dhc, dhs, nullptr);
    if (!st) st = f.sync(ctx, nullptr);
    const int32_t sc = st;
    if (!st) st = f.to_host(ctx, Y.data(), dy, 4 * n_tok * n_embd, nullptr);
    if (!st) st = f.to_host(ctx, HC.data(), dhc, n_tok * n_ff, nullptr);
    if (!st) st = f.to_host(ctx, HS.data(), dhs, 8 * n_tok * nbh, nullptr);
    put(fo, sc);
    put_arr(fo, Y);
    put_arr(fo, HC);
    put_arr(fo, HS);
    std::fclose(fo);
    f.dev_free(ctx, stage);
    for (ah_tensor *w : t) f.free_tensor(ctx, w);
    std::printf("ENGINE projections %s, ffn %s, group %s, column ffn %s\n", rust_error(sp), rust_error(sf),
                rust_error(sg), rust_error(sc));
    return st == AH_OK ? 0 : 4;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s LIB status|probe|run|engine IN OUT\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[2];
    void *lib = dlopen(argv[1], RTLD_NOW);
    if (!lib) {
        std::printf("SKIP %s not found\n", argv[1]);
        return 0;
    }
    Fns f{};
    if (!resolve(lib, f)) return 0;
    if (mode == "status") {
        for (int32_t st = 0; st <= 26; ++st) std::printf("%d %s | %s\n", st, rust_error(st), f.status_str(st));
        dlclose(lib);
        return 0;
    }
    ah_ctx *ctx = nullptr;
    const int32_t si = f.init(0, &ctx);
    if (si != AH_OK) {
        std::printf("SKIP ah_init: %s (status %d, %s)\n", f.status_str(si), si, rust_error(si));
        dlclose(lib);
        return 0;
    }
    int rc = 0;
    if (mode == "probe") {
        std::printf("DEVICE ok\n");
    } else if (mode == "run" && argc >= 5) {
        rc = run_case(f, ctx, argv[3], argv[4]);
    } else if (mode == "engine" && argc >= 5) {
        rc = run_engine(f, ctx, argv[3], argv[4]);
    } else {
        rc = 2;
    }
    f.destroy(ctx);
    dlclose(lib);
    return rc;
}
