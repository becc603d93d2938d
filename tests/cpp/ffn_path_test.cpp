// ffn_path_test.cpp -- drives the C++ host layer (neutron-star_amd/host/ffn_path.hpp)
// the way the reference engine drives its FFN helpers (metal_engine.mm:562-576):
// decode FFN block + lm-head, then a prefill FFN block in both accumulation
// modes, each checked against the CPU oracle; then the error convention
// (std::runtime_error); then the whole load chain of the engine: a GGUF image is
// converted to .nsmffn (convert_metal_ffn), mapped and validated (MetalFfnFile),
// uploaded with the CDNA4 re-tile (WeightImage), and run through ffn_block with
// the per-layer accumulation-mode rule of mm:565.  Exit status 0 = pass.  Built by __graft_entry__.build()
// and run by tests/test_gpu_cpp_path.py on the GPU.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <vector>

#include <unistd.h>

#include "ffn_path.hpp"
#include "gguf_file.hpp"
#include "nsmffn_file.hpp"
#include "ns_oracle.h"

using namespace neutron::amd;

namespace {
int failures = 0;

void expect(bool ok, const char *what) {
    std::printf("%s: %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok) ++failures;
}

// max over rows of max|got-ref| / max|ref|
double rel_err(const std::vector<float> &got, const std::vector<float> &ref, size_t rows, size_t cols) {
    double worst = 0;
    for (size_t r = 0; r < rows; ++r) {
        double num = 0, den = 1e-30;
        for (size_t c = 0; c < cols; ++c) {
            num = std::fmax(num, std::fabs(double(got[r * cols + c]) - ref[r * cols + c]));
            den = std::fmax(den, std::fabs(double(ref[r * cols + c])));
        }
        worst = std::fmax(worst, num / den);
    }
    return worst;
}

std::vector<uint8_t> synth(TensorType t, uint64_t seed, uint64_t rows, uint64_t cols) {
    const size_t bs = t == TensorType::Q4_K ? 144 : 210;
    std::vector<uint8_t> v(rows * (cols / 256) * bs);
    check(ns_synth_blocks(int(t), seed, 0, rows * (cols / 256), v.data(), 4));
    return v;
}

template <class T>
T *dev(const std::vector<T> &h) {
    T *p = nullptr;
    if (hipMalloc(&p, h.size() * sizeof(T)) != hipSuccess) throw std::runtime_error("hipMalloc");
    if (hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return p;
}
template <class T>
std::vector<T> host(const T *p, size_t n) {
    std::vector<T> h(n);
    if (hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess) throw std::runtime_error("hipMemcpy");
    return h;
}
}  // namespace

int main() {
    const uint64_t D = 768, F = 512, V = 1024, B = 70;
    hipStream_t s = nullptr;
    if (hipStreamCreate(&s) != hipSuccess) return 2;

    // Tensors as the engine sees them: gate/up Q4_K [F][D], down Q6_K [D][F],
    // token embedding (lm-head) Q6_K [V][D] row-major.
    Tensor gate{"blk.0.ffn_gate.weight", {D, F}, TensorType::Q4_K, 0, F * (D / 256) * 144};
    Tensor up{"blk.0.ffn_up.weight", {D, F}, TensorType::Q4_K, 1, F * (D / 256) * 144};
    Tensor down{"blk.0.ffn_down.weight", {F, D}, TensorType::Q6_K, 2, D * (F / 256) * 210};
    Tensor embd{"token_embd.weight", {D, V}, TensorType::Q6_K, 3, V * (D / 256) * 210};
    const auto hg = synth(gate.type, 11, F, D), hu = synth(up.type, 12, F, D);
    const auto hd = synth(down.type, 13, D, F), he = synth(embd.type, 14, V, D);
    // the FFN tensors arrive in the .nsmffn order (as neutron-convert-metal-ffn writes them)
    auto nsm = [&](const std::vector<uint8_t> &rm, const Tensor &t) {
        std::vector<uint8_t> o(rm.size());
        check(ns_retile(rm.data(), o.data(), int(t.type), uint32_t(t.shape[0]), uint32_t(t.shape[1]),
                        NS_LAYOUT_ROW_MAJOR, NS_LAYOUT_NSMFFN));
        return o;
    };
    WeightImage img;
    uint64_t off[4], total = 0;
    for (int i = 0; i < 4; ++i) {
        off[i] = total;
        const Tensor &t = i == 0 ? gate : i == 1 ? up : i == 2 ? down : embd;
        total += (t.bytes + 255) / 256 * 256;
    }
    img.allocate(total);
    img.upload(gate, nsm(hg, gate).data(), off[0], Layout::Nsmffn, true, s);
    img.upload(up, nsm(hu, up).data(), off[1], Layout::Nsmffn, true, s);
    img.upload(down, nsm(hd, down).data(), off[2], Layout::Nsmffn, true, s);
    img.upload(embd, he.data(), off[3], Layout::RowMajor, false, s);
    expect(img.layout(gate) == Layout::Cdna4 && img.layout(embd) == Layout::RowMajor, "conversion at load time");
    FfnPath path(img);

    // ---- decode (mm:571-576): gate/up GeGLU, down GEMV, lm-head GEMV
    std::vector<float> x(D), xe(D);
    check(ns_synth_normal_f32(21, 0, D, x.data(), 4));
    check(ns_synth_normal_f32(22, 0, D, xe.data(), 4));
    float *dx = dev(x), *dxe = dev(xe), *dh = dev(std::vector<float>(F)), *dy = dev(std::vector<float>(D));
    float *dl = dev(std::vector<float>(V));
    path.gate_up_geglu_decode(s, gate, up, dx, dh);
    path.ffn_down(s, down, dh, dy, 1, false);
    path.matmul(s, embd, dxe, dl, 1);
    if (hipStreamSynchronize(s) != hipSuccess) return 3;
    const auto h = host(dh, F), y = host(dy, D), l = host(dl, V);
    std::vector<float> h_ref(F), y_ref(D), l_ref(V);
    nso_gate_up_geglu(NSO_ROW_MAJOR, hg.data(), hu.data(), D, F, x.data(), h_ref.data(), 4);
    nso_gemv(NSO_Q6_K, NSO_ROW_MAJOR, hd.data(), F, D, h.data(), y_ref.data(), 4);
    nso_gemv(NSO_Q6_K, NSO_ROW_MAJOR, he.data(), D, V, xe.data(), l_ref.data(), 4);
    expect(rel_err(h, h_ref, 1, F) <= 1e-3, "decode gate/up GeGLU within 1e-3");
    expect(rel_err(y, y_ref, 1, D) <= 1e-3, "decode down GEMV within 1e-3");
    expect(rel_err(l, l_ref, 1, V) <= 1e-3, "lm-head GEMV (row-major) within 1e-3");

    // ---- decode of 2-4 fp32 tokens (mm:570-573): matmul(gate), matmul(up), gemma_geglu, down
    for (uint32_t bt : {2u, 4u}) {
        std::vector<float> xb(bt * D);
        check(ns_synth_normal_f32(24 + bt, 0, bt * D, xb.data(), 4));
        float *dxb = dev(xb), *dhb = dev(std::vector<float>(bt * F)), *dyb = dev(std::vector<float>(bt * D));
        path.ffn_block(s, gate, up, down, dxb, dhb, dyb, bt, /*prefill=*/false, /*swa=*/true, /*exact_ffn=*/false);
        bool threw_status = false;
        try { path.finish(s); } catch (const std::runtime_error &) { threw_status = true; }
        expect(!threw_status, "finish() after a decode block reports no timed-out wait");
        const auto hb = host(dhb, bt * F), yb = host(dyb, bt * D);
        std::vector<float> hb_ref(bt * F), yb_ref(bt * D);
        for (uint32_t t = 0; t < bt; ++t) {
            nso_gate_up_geglu(NSO_ROW_MAJOR, hg.data(), hu.data(), D, F, xb.data() + t * D, hb_ref.data() + t * F, 4);
            nso_gemv(NSO_Q6_K, NSO_ROW_MAJOR, hd.data(), F, D, hb.data() + t * F, yb_ref.data() + t * D, 4);
        }
        expect(rel_err(hb, hb_ref, bt, F) <= 1e-3, bt == 2 ? "decode block, 2 tokens: h within 1e-3" : "decode block, 4 tokens: h within 1e-3");
        expect(rel_err(yb, yb_ref, bt, D) <= 1e-3, bt == 2 ? "decode block, 2 tokens: y within 1e-3" : "decode block, 4 tokens: y within 1e-3");
        (void)hipFree(dxb);
        (void)hipFree(dhb);
        (void)hipFree(dyb);
    }

    // ---- prefill (mm:563-573), both accumulation modes
    std::vector<uint16_t> xp(B * D);
    check(ns_synth_normal_f16(23, 0, B * D, xp.data(), 4));
    uint16_t *dxp = dev(xp), *dhp = dev(std::vector<uint16_t>(B * F));
    float *dyp = dev(std::vector<float>(B * D));
    for (int fast = 0; fast < 2; ++fast) {
        path.gate_up_geglu_rm32(s, gate, up, dxp, dhp, uint32_t(B), fast != 0);
        path.ffn_down(s, down, dhp, dyp, uint32_t(B), true, fast != 0);
        if (hipStreamSynchronize(s) != hipSuccess) return 3;
        const auto hp16 = host(dhp, B * F);
        const auto yp = host(dyp, B * D);
        std::vector<float> hp(B * F), hp_ref(B * F), yp_ref(B * D);
        for (size_t i = 0; i < hp.size(); ++i) hp[i] = nso_f16_to_f32(hp16[i]);
        nso_gate_up_geglu_prefill(NSO_ROW_MAJOR, hg.data(), hu.data(), D, F, B, xp.data(), 0, hp_ref.data(), 4);
        nso_gemm(NSO_Q6_K, NSO_ROW_MAJOR, hd.data(), F, D, B, hp16.data(), 0, yp_ref.data(), 4);
        const double tol = fast ? 1e-2 : 1e-3;
        expect(rel_err(hp, hp_ref, B, F) <= tol, fast ? "prefill gate/up FP16 mode within 1e-2" : "prefill gate/up FP32 mode within 1e-3");
        expect(rel_err(yp, yp_ref, B, D) <= tol, fast ? "prefill down FP16 mode within 1e-2" : "prefill down FP32 mode within 1e-3");
    }

    // ---- errors surface as std::runtime_error (mm:231-243 convention)
    Tensor missing{"blk.9.ffn_up.weight", {D, F}, TensorType::Q4_K, 99, 0};
    bool threw = false;
    try { path.matmul(s, missing, dx, dh, 1); } catch (const std::runtime_error &) { threw = true; }
    expect(threw, "unknown tensor throws");
    threw = false;
    try { path.gate_up_geglu_decode(s, gate, down, dx, dh); } catch (const std::runtime_error &) { threw = true; }
    expect(threw, "gate/up shape mismatch throws");
    threw = false;
    try { path.matmul(s, gate, dx, dh, 0); } catch (const std::runtime_error &e) { threw = std::strstr(e.what(), "batch") != nullptr; }
    expect(threw, "zero batch throws with the C ABI message");

    // ---- load chain: GGUF v3 file -> GGUF -> .nsmffn -> MetalFfnFile -> WeightImage -> ffn_block
    {
        const Tensor *ts[4] = {&gate, &up, &down, &embd};
        const std::vector<uint8_t> *hs[4] = {&hg, &hu, &hd, &he};
        std::vector<ns_tensor_desc> table;
        uint64_t pos = 0;
        for (int i = 0; i < 4; ++i) {
            const Tensor &t = *ts[i];
            const bool ffn = i < 3;
            table.push_back({pos, t.bytes, uint32_t(t.type), uint32_t(t.shape[0]), uint32_t(t.shape[1]),
                             ffn ? 0u : NS_FFN_NONE, ffn ? uint32_t(i) : NS_FFN_NONE, 0});
            pos += (t.bytes + 31) / 32 * 32;
        }
        // GGUF v3 header: one metadata entry (general.alignment = 65536, so the data section
        // starts past the .nsmffn header page) and the four tensor entries
        std::vector<uint8_t> gguf;
        auto put = [&](const void *p, size_t n) {
            gguf.insert(gguf.end(), static_cast<const uint8_t *>(p), static_cast<const uint8_t *>(p) + n);
        };
        auto put32 = [&](uint32_t v) { put(&v, 4); };
        auto put64 = [&](uint64_t v) { put(&v, 8); };
        auto putstr = [&](const std::string &s) { put64(s.size()); put(s.data(), s.size()); };
        put("GGUF", 4); put32(3); put64(4); put64(1);
        putstr("general.alignment"); put32(4 /* u32 */); put32(65536);
        for (int i = 0; i < 4; ++i) {
            putstr(ts[i]->name); put32(2); put64(ts[i]->shape[0]); put64(ts[i]->shape[1]);
            put32(uint32_t(ts[i]->type)); put64(table[i].source_offset);
        }
        const uint64_t data_offset = 65536;
        for (size_t i = gguf.size(); i < data_offset; ++i) gguf.push_back(uint8_t(i * 131 + 7));
        gguf.resize(data_offset + pos, 0);
        for (int i = 0; i < 4; ++i)
            std::memcpy(gguf.data() + data_offset + table[i].source_offset, hs[i]->data(), hs[i]->size());
        const std::string gfile = "/tmp/ffn_path_test_" + std::to_string(getpid()) + ".gguf";
        {
            FILE *fo = std::fopen(gfile.c_str(), "wb");
            expect(fo && std::fwrite(gguf.data(), 1, gguf.size(), fo) == gguf.size(), "GGUF file written");
            if (fo) std::fclose(fo);
        }
        GGUF gg(gfile, false);
        expect(gg.data_offset() == data_offset && gg.file_size() == gguf.size() && gg.meta_u64("general.alignment") == 65536,
               "GGUF: data offset, size and alignment");
        expect(gg.tensor("blk.0.ffn_down.weight").bytes == down.bytes && gg.has_tensor("token_embd.weight") &&
                   !gg.has_tensor("blk.0.attn_q.weight"),
               "GGUF: tensor lookup");
        const std::vector<ns_tensor_desc> gt = gg.ffn_tensor_table();
        bool same = gt.size() == table.size();
        for (size_t i = 0; same && i < gt.size(); ++i)
            same = gt[i].source_offset == table[i].source_offset && gt[i].bytes == table[i].bytes &&
                   gt[i].type == table[i].type && gt[i].layer == table[i].layer && gt[i].kind == table[i].kind;
        expect(same, "GGUF: the FFN tensor table from the file equals the engine's");
        threw = false;
        try { (void)gg.tensor("blk.0.attn_q.weight"); } catch (const std::runtime_error &e) { threw = std::strstr(e.what(), "missing tensor") != nullptr; }
        expect(threw, "GGUF: missing tensor throws the reference's message");
        std::remove(gfile.c_str());
        const std::string file = "/tmp/ffn_path_test_" + std::to_string(getpid()) + ".nsmffn";
        convert_metal_ffn(file, gguf.data(), gguf.size(), data_offset, gt);
        const uint64_t fp = metal_ffn_fingerprint(gguf.data(), data_offset, gguf.size());
        MetalFfnFile mf(file, gguf.size(), fp, table);
        expect(mf.reordered(table[0].source_offset) && !mf.reordered(table[3].source_offset),
               "MetalFfnFile: FFN tensors reordered, embedding not");
        // the engine's tensors are keyed by their GGUF offset
        Tensor g2 = gate, u2 = up, d2 = down, e2 = embd;
        Tensor *t2[4] = {&g2, &u2, &d2, &e2};
        for (int i = 0; i < 4; ++i) t2[i]->offset = table[i].source_offset;
        WeightImage img2;
        img2.allocate(mf.file_size());
        for (int i = 0; i < 4; ++i) {
            const uint64_t o = mf.offset(t2[i]->offset);
            img2.upload(*t2[i], mf.mapped_data() + o, o, mf.reordered(t2[i]->offset) ? Layout::Nsmffn : Layout::RowMajor,
                        true, s);
        }
        FfnPath p2(img2);
        // decode block (always FP32), then the next layer's RMSNorm (rms, mm:563) with unit
        // weights: unit RMS; and rms fused into the next gate/up equals rms then gate/up
        float *dx2 = dev(std::vector<float>(D));
        float *dones = dev(std::vector<float>(D, 1.0f));
        float *dh2 = dev(std::vector<float>(F));
        float *dh3 = dev(std::vector<float>(F));
        p2.ffn_block(s, g2, u2, d2, dx, dh, dy, 1, /*prefill=*/false, /*swa=*/true, /*exact_ffn=*/false);
        p2.rms(s, dy, dx2, dones, uint32_t(D), 1, 0.0f);
        p2.gate_up_geglu_decode(s, g2, u2, dx2, dh2);
        p2.rms_gate_up_geglu_decode(s, g2, u2, dy, dones, 0.0f, dh3);
        if (hipStreamSynchronize(s) != hipSuccess) return 3;
        const auto yb = host(dy, D), xr = host(dx2, D);
        expect(rel_err(yb, y_ref, 1, D) <= 1e-3 && rel_err(host(dh, F), h_ref, 1, F) <= 1e-3,
               "ffn_block decode from the .nsmffn file within 1e-3");
        double ss = 0;
        for (float v : xr) ss += double(v) * v;
        expect(std::fabs(std::sqrt(ss / D) - 1.0) < 1e-5, "rms with unit weights: unit RMS");
        expect(rel_err(host(dh3, F), host(dh2, F), 1, F) <= 1e-5, "rms fused into gate/up == rms then gate/up");
        (void)hipFree(dones); (void)hipFree(dh2); (void)hipFree(dh3);
        // prefill block: a local (swa) layer runs FP16 mode, a global one or --exact-ffn FP32 (mm:565)
        for (int c = 0; c < 3; ++c) {
            const bool swa = c != 1, exact = c == 2;
            p2.ffn_block(s, g2, u2, d2, dxp, dhp, dyp, uint32_t(B), true, swa, exact);
            if (hipStreamSynchronize(s) != hipSuccess) return 3;
            const auto yq = host(dyp, B * D);
            bool f16p = true;
            for (float v : yq) {
                uint32_t bits;
                std::memcpy(&bits, &v, 4);
                f16p = f16p && (bits & 0x1FFFu) == 0;
            }
            const bool fast = swa && !exact;
            expect(f16p == fast, fast ? "local layer: FP16 mode (fp16-precision outputs)"
                                      : "global layer / exact_ffn: FP32 mode (full-precision outputs)");
        }
        (void)hipFree(dx2);
        std::remove(file.c_str());
    }

    (void)hipFree(dx); (void)hipFree(dxe); (void)hipFree(dh); (void)hipFree(dy); (void)hipFree(dl);
    (void)hipFree(dxp); (void)hipFree(dhp); (void)hipFree(dyp);
    (void)hipStreamDestroy(s);
    std::printf("%s (%d failures)\n", failures ? "FAILED" : "PASSED", failures);
    return failures ? 1 : 0;
}
