// Compiled torch binding of the decode path: class Decoder with the signature
// of the reference's bindings/torch_decode.cu:14-81 (plan(seq_lens, num_ctas),
// run(q, k_cache, v_cache, block_table, seq_lens_dev, k_scale, v_scale),
// num_ctas, num_segments), over the C ABI of libpa_decode.so. It runs on the
// current torch stream. Argument errors raise RuntimeError (TORCH_CHECK), the
// library's invalid-argument / length errors ValueError (pybind11's mapping of
// std::invalid_argument / std::length_error, as the reference's make_plan
// throws them), device errors RuntimeError.
//
// plan() builds the launch parameters that stay fixed between calls (shapes,
// softmax scale, the bound device plan); run() checks its tensors, allocates
// the output and fills in the per-call pointers and scales, then launches.

#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <cmath>
#include <stdexcept>
#include <string>

#include "pa_decode.h"

namespace {

void check_status(pa_status s) {
    if (s == PA_OK) return;
    const std::string msg = pa_last_error();
    if (s == PA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    if (s == PA_ERR_LENGTH) throw std::length_error(msg);
    throw std::runtime_error("paged decode: " + msg);
}

class Decoder {
public:
    Decoder(int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size, bool fp8)
        : hq_(static_cast<int>(num_q_heads)),
          hkv_(static_cast<int>(num_kv_heads)),
          dim_(static_cast<int>(head_dim)),
          page_(static_cast<int>(page_size)),
          dtype_(fp8 ? PA_KV_FP8_E4M3 : PA_KV_FP16) {
        check_status(pa_device_plan_create(&dplan_));
    }
    ~Decoder() {
        pa_plan_destroy(plan_);
        pa_device_plan_destroy(dplan_);
    }
    Decoder(const Decoder&)            = delete;
    Decoder& operator=(const Decoder&) = delete;

    // torch_decode.cu:21-27: seq_lens is a CPU int32 tensor [batch].
    void plan(const torch::Tensor& seq_lens, int64_t num_ctas) {
        TORCH_CHECK(seq_lens.device().is_cpu() && seq_lens.scalar_type() == torch::kInt32,
                    "seq_lens must be a CPU int32 tensor");
        const torch::Tensor lens = seq_lens.contiguous();
        const int batch = static_cast<int>(lens.numel());
        pa_plan* next = nullptr;
        check_status(pa_plan_build(dtype_, lens.data_ptr<int32_t>(), batch, hq_, hkv_, dim_,
                                   static_cast<int>(num_ctas), &next));
        pa_plan_destroy(plan_);
        plan_ = next;
        const int device = c10::hip::current_device();
        check_status(pa_device_plan_upload(dplan_, plan_, hkv_ > 0 ? hq_ / hkv_ : 0, dim_,
                                           c10::hip::getCurrentHIPStream(device).stream()));
        int max_len = 0;
        const int32_t* l = lens.data_ptr<int32_t>();
        for (int i = 0; i < batch; ++i) max_len = std::max(max_len, l[i]);
        table_cols_ = (max_len + page_ - 1) / page_;
        batch_      = batch;
        tmpl_       = pa_decode_params{};
        tmpl_.batch        = batch;
        tmpl_.num_q_heads  = hq_;
        tmpl_.num_kv_heads = hkv_;
        tmpl_.head_dim     = dim_;
        tmpl_.page_size    = page_;
        tmpl_.sm_scale     = 1.0f / std::sqrt(static_cast<float>(dim_));
        check_status(pa_device_plan_bind(dplan_, &tmpl_));
    }

    // torch_decode.cu:31-59. q [batch, Hq, D] fp16; caches [pages, Hkv, P, D]
    // fp16 or one-byte FP8; block_table [batch, >= ceil(max len / P)] int32.
    torch::Tensor run(const torch::Tensor& q, const torch::Tensor& k_cache, const torch::Tensor& v_cache,
                      const torch::Tensor& block_table, const torch::Tensor& seq_lens_dev, double k_scale,
                      double v_scale) {
        TORCH_CHECK(q.is_cuda() && q.scalar_type() == torch::kHalf && q.is_contiguous(),
                    "q must be a contiguous CUDA fp16 tensor");
        TORCH_CHECK(k_cache.is_contiguous() && v_cache.is_contiguous() && block_table.is_contiguous(),
                    "caches and block_table must be contiguous");
        TORCH_CHECK(plan_ != nullptr && q.size(0) == batch_, "q batch does not match the plan");
        TORCH_CHECK(block_table.scalar_type() == torch::kInt32, "block_table must be int32");
        // Shape checks beyond the reference's: a mismatch would otherwise
        // become out-of-range device reads.
        TORCH_CHECK(q.dim() == 3 && q.size(1) == hq_ && q.size(2) == dim_, "q must be [batch, num_q_heads, head_dim]");
        const int64_t elem = dtype_ == PA_KV_FP16 ? 2 : 1;
        for (const torch::Tensor* c : {&k_cache, &v_cache})
            TORCH_CHECK(c->is_cuda() && c->dim() == 4 && c->size(1) == hkv_ && c->size(2) == page_ &&
                            c->size(3) == dim_ && c->element_size() == elem,
                        "k_cache / v_cache must be CUDA [pages, num_kv_heads, page_size, head_dim] tensors of ",
                        elem == 2 ? "fp16" : "one-byte FP8", " elements");
        TORCH_CHECK(block_table.is_cuda() && block_table.dim() == 2 && block_table.size(0) >= batch_ &&
                        block_table.size(1) >= table_cols_,
                    "block_table must be a CUDA [batch, >= ceil(max seq_len / page_size)] tensor");
        TORCH_CHECK(seq_lens_dev.is_cuda() && seq_lens_dev.scalar_type() == torch::kInt32,
                    "seq_lens must be a CUDA int32 tensor");
        torch::Tensor out = torch::empty_like(q);
        pa_decode_params p = tmpl_;
        p.q                  = static_cast<const uint16_t*>(q.data_ptr());
        p.out                = static_cast<uint16_t*>(out.data_ptr());
        p.k_cache            = k_cache.data_ptr();
        p.v_cache            = v_cache.data_ptr();
        p.block_table        = block_table.data_ptr<int32_t>();
        p.seq_lens           = seq_lens_dev.data_ptr<int32_t>();
        p.block_table_stride = static_cast<int32_t>(block_table.size(1));
        p.k_scale            = static_cast<float>(k_scale);
        p.v_scale            = static_cast<float>(v_scale);
        check_status(pa_decode(dtype_, &p, c10::hip::getCurrentHIPStream(q.get_device()).stream()));
        return out;
    }

    int64_t num_ctas() const { return pa_plan_num_ctas(plan_); }
    int64_t num_segments() const { return pa_plan_num_segments(plan_); }

private:
    int             hq_, hkv_, dim_, page_;
    int             dtype_;
    int             batch_      = 0;
    int             table_cols_ = 0;
    pa_plan*        plan_       = nullptr;
    pa_device_plan* dplan_      = nullptr;
    pa_decode_params tmpl_{};
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Compiled torch binding of the MI355X paged decode path (libpa_decode.so)";
    pybind11::class_<Decoder>(m, "Decoder")
        .def(pybind11::init<int64_t, int64_t, int64_t, int64_t, bool>(), pybind11::arg("num_q_heads"),
             pybind11::arg("num_kv_heads"), pybind11::arg("head_dim"), pybind11::arg("page_size"),
             pybind11::arg("fp8"))
        .def("plan", &Decoder::plan, pybind11::arg("seq_lens"), pybind11::arg("num_ctas") = 0)
        .def("run", &Decoder::run, pybind11::arg("q"), pybind11::arg("k_cache"), pybind11::arg("v_cache"),
             pybind11::arg("block_table"), pybind11::arg("seq_lens_dev"), pybind11::arg("k_scale"),
             pybind11::arg("v_scale"))
        .def_property_readonly("num_ctas", &Decoder::num_ctas)
        .def_property_readonly("num_segments", &Decoder::num_segments);
}
