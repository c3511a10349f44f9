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
           sym(lib, "ah_last_refusal_bits", f.refusal_bits) && sym(lib, "ah_probe_mfma_peak", f.probe);
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

}  // namespace

int main(int argc, char **argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s LIB status|probe|run IN OUT\n", argv[0]);
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
    } else {
        rc = 2;
    }
    f.destroy(ctx);
    dlclose(lib);
    return rc;
}
