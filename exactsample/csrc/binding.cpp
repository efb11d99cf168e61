// PyTorch-ROCm custom op exactsample::verify_out on top of the C ABI.
//
// Replaces the reference's op binding (csrc/bindings.cpp:45-146): the same
// schema string, the same structural checks and the same error messages
// (callers and tests match on them), then one es_launch on the current HIP
// stream. All checks run on the host before anything is enqueued; the kernels
// report numerical problems per request instead.
#include <ATen/ATen.h>
// PyTorch-ROCm tensors report the "cuda" device type; these are its HIP guard and stream for them.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <cstdint>
#include <limits>
#include <numeric>
#include <string>
#include <vector>

#include "exactsample_amd.h"

namespace {
using at::Tensor;
constexpr int64_t kInt32Max = std::numeric_limits<int32_t>::max();

int32_t logits_code(const Tensor& t) {
  const at::ScalarType s = t.scalar_type();
  if (s == at::kFloat) return ES_F32;
  if (s == at::kBFloat16) return ES_BF16;
  if (s == at::kHalf) return ES_F16;
  if (s == at::kDouble) return ES_F64;
  TORCH_CHECK(false, "exactsample logits require float16/bfloat16/float32/float64");
}

// The byte range [first, last) that a view with non-negative strides can touch.
struct ByteRange {
  uintptr_t first = 0, last = 0;
  bool empty = true;
};
ByteRange byte_range(const Tensor& t) {
  ByteRange r;
  if (t.numel() == 0) return r;
  int64_t reach = 1;
  for (int64_t d = 0; d < t.dim(); ++d) reach += (t.size(d) - 1) * t.stride(d);
  r.first = reinterpret_cast<uintptr_t>(t.const_data_ptr());
  r.last = r.first + uintptr_t(reach) * uintptr_t(t.element_size());
  r.empty = false;
  return r;
}
bool share_bytes(const ByteRange& x, const ByteRange& y) {
  return !x.empty && !y.empty && x.first < y.last && y.first < x.last;
}

// Whether two different indices of a (1-D or 2-D) view name one element. For
// strides s0, s1 with g = gcd(s0, s1), the index steps (di, dj) with
// di * s0 == dj * s1 are the multiples of (s1 / g, s0 / g), so a collision
// needs both s1 / g < size(0) and s0 / g < size(1).
bool aliases_itself(const Tensor& t) {
  if (t.numel() < 2) return false;
  for (int64_t d = 0; d < t.dim(); ++d)
    if (t.size(d) > 1 && t.stride(d) == 0) return true;
  if (t.dim() < 2 || t.size(0) == 1 || t.size(1) == 1) return false;
  const int64_t g = std::gcd(t.stride(0), t.stride(1));
  return t.stride(1) / g < t.size(0) && t.stride(0) / g < t.size(1);
}

// One call's tensors after their checks, in the order the C ABI wants them.
class Call {
 public:
  explicit Call(const Tensor& logits) : device_(logits.device()) {
    TORCH_CHECK(logits.is_cuda() && logits.dim() == 2, "target_logits must be a 2D CUDA tensor");
    rows_ = logits.size(0);
    vocab_ = logits.size(1);
  }

  // Device, element type, rank and non-negative strides of one argument.
  void expect(const Tensor& t, at::ScalarType type, int64_t rank, const char* what) const {
    TORCH_CHECK(t.device() == device_ && t.scalar_type() == type && t.dim() == rank, what,
                " has wrong device, dtype or rank");
    for (int64_t d = 0; d < rank; ++d) TORCH_CHECK(t.stride(d) >= 0, what, " has a negative stride");
  }
  void read(const Tensor& t) { reads_.push_back(t); }
  void write(const Tensor& t) { writes_.push_back(t); }

  // Outputs never overlap themselves, an input, or an earlier output.
  void check_aliasing() const {
    std::vector<ByteRange> in;
    for (const Tensor& t : reads_) in.push_back(byte_range(t));
    std::vector<ByteRange> out;
    for (const Tensor& t : writes_) {
      TORCH_CHECK(!aliases_itself(t), "output has overlapping strides");
      const ByteRange r = byte_range(t);
      for (const ByteRange& x : in) TORCH_CHECK(!share_bytes(r, x), "exactsample input/output aliasing is forbidden");
      for (const ByteRange& x : out) TORCH_CHECK(!share_bytes(r, x), "exactsample outputs alias");
      out.push_back(r);
    }
  }

  at::Device device() const { return device_; }
  int64_t rows() const { return rows_; }
  int64_t vocab() const { return vocab_; }

 private:
  at::Device device_;
  int64_t rows_ = 0, vocab_ = 0;
  std::vector<Tensor> reads_, writes_;
};

es_matrix as_matrix(const Tensor& t) {
  es_matrix m{};
  m.data = t.const_data_ptr();
  m.s0 = t.stride(0);
  m.s1 = t.stride(1);
  m.dtype = logits_code(t);
  return m;
}
es_vec_i64 as_i64(const Tensor& t) { return es_vec_i64{t.const_data_ptr<int64_t>(), t.stride(0)}; }
es_vec_f64 as_f64(const Tensor& t) { return es_vec_f64{t.const_data_ptr<double>(), t.stride(0)}; }

void verify_out(const Tensor& target_logits, const Tensor& cu_rows, const Tensor& draft_ids,
                const c10::optional<Tensor>& draft_logits, const Tensor& temperature, const Tensor& top_k,
                const Tensor& top_p, const Tensor& min_p, const Tensor& draft_kind, const Tensor& seeds,
                const Tensor& stream_ids, const Tensor& positions, const c10::optional<Tensor>& mask,
                Tensor workspace, Tensor tokens, Tensor accepted_len, Tensor status, Tensor path_used,
                int64_t mode, int64_t dispatch, int64_t max_draft, int64_t list_max) {
  Call call(target_logits);
  const int64_t rows = call.rows(), vocab = call.vocab();

  // Shape of the batch and the scalar options.
  call.expect(cu_rows, at::kLong, 1, "cu_rows");
  TORCH_CHECK(cu_rows.numel() >= 1, "cu_rows must contain an endpoint");
  const int64_t requests = cu_rows.numel() - 1;
  TORCH_CHECK(requests != 0 || rows == 0, "an empty request batch cannot contain target rows");
  TORCH_CHECK(vocab > 0 && vocab <= kInt32Max && rows <= kInt32Max && requests <= kInt32Max,
              "exactsample dimensions exceed int32 kernel indexing");
  TORCH_CHECK(rows <= 65535, "exactsample supports at most 65535 target rows per call");
  TORCH_CHECK(max_draft >= 0 && max_draft < kInt32Max, "invalid max_draft");
  TORCH_CHECK(mode >= 0 && mode <= 1 && dispatch >= 0 && dispatch <= 2, "invalid mode/dispatch");
  TORCH_CHECK(list_max >= 0 && list_max <= 256, "list_max must be in [0, 256]");
  call.expect(draft_ids, at::kLong, 2, "draft_ids");
  TORCH_CHECK(draft_ids.size(0) == requests && draft_ids.size(1) >= max_draft, "draft_ids capacity mismatch");

  // Per-request parameters, then per-row positions.
  for (const Tensor* t : {&temperature, &top_p, &min_p}) {
    call.expect(*t, at::kDouble, 1, "floating request parameter");
    TORCH_CHECK(t->numel() == requests, "request parameter length mismatch");
  }
  for (const Tensor* t : {&top_k, &draft_kind, &seeds, &stream_ids}) {
    call.expect(*t, at::kLong, 1, "integer request parameter");
    TORCH_CHECK(t->numel() == requests, "request parameter length mismatch");
  }
  call.expect(positions, at::kLong, 1, "positions");
  TORCH_CHECK(positions.numel() == rows, "positions must be per target row");
  for (const Tensor* t : {&target_logits, &cu_rows, &draft_ids, &temperature, &top_k, &top_p, &min_p, &draft_kind,
                          &seeds, &stream_ids, &positions})
    call.read(*t);

  es_arguments a{};
  a.target = as_matrix(target_logits);
  a.draft = es_matrix{nullptr, 0, 0, a.target.dtype, 0};
  if (draft_logits) {
    const Tensor& q = *draft_logits;
    TORCH_CHECK(q.device() == call.device() && q.dim() == 2 && q.sizes() == target_logits.sizes(),
                "draft_logits shape/device mismatch");
    TORCH_CHECK(q.scalar_type() == target_logits.scalar_type(), "draft_logits must have the target_logits dtype");
    a.draft = as_matrix(q);
    call.read(q);
  }
  if (mask) {
    const Tensor& m = *mask;
    call.expect(m, at::kInt, 2, "mask");
    TORCH_CHECK(m.size(0) == rows && m.size(1) == (vocab + 31) / 32, "mask shape mismatch");
    a.mask = m.const_data_ptr<int32_t>();
    a.mask_s0 = m.stride(0);
    a.mask_s1 = m.stride(1);
    call.read(m);
  }

  // Workspace and outputs.
  call.expect(workspace, at::kByte, 1, "workspace");
  TORCH_CHECK(workspace.is_contiguous(), "workspace must be contiguous");
  const size_t need = es_workspace_size(rows, vocab, dispatch == 1 ? 1 : 0);
  TORCH_CHECK(need != 0, "workspace size overflow");
  TORCH_CHECK(uint64_t(workspace.numel()) >= need,
              dispatch == 1 ? "workspace capacity exceeded (the reference path needs a plan made with reference=True)"
                            : "workspace capacity exceeded");
  TORCH_CHECK(reinterpret_cast<uintptr_t>(workspace.data_ptr()) % 8 == 0, "workspace alignment must be 8 bytes");
  call.expect(tokens, at::kLong, 2, "tokens");
  TORCH_CHECK(tokens.size(0) >= requests && tokens.size(1) >= max_draft + 1, "tokens capacity exceeded");
  for (const Tensor* t : {&accepted_len, &status, &path_used}) {
    call.expect(*t, at::kInt, 1, "output");
    TORCH_CHECK(t->numel() >= requests, "output capacity exceeded");
  }
  for (const Tensor* t : {&workspace, &tokens, &accepted_len, &status, &path_used}) call.write(*t);
  call.check_aliasing();

  a.cu_rows = as_i64(cu_rows);
  a.top_k = as_i64(top_k);
  a.draft_kind = as_i64(draft_kind);
  a.seed = as_i64(seeds);
  a.stream = as_i64(stream_ids);
  a.position = as_i64(positions);
  a.temperature = as_f64(temperature);
  a.top_p = as_f64(top_p);
  a.min_p = as_f64(min_p);
  a.draft_ids = draft_ids.const_data_ptr<int64_t>();
  a.draft_s0 = draft_ids.stride(0);
  a.draft_s1 = draft_ids.stride(1);
  a.tokens = tokens.data_ptr<int64_t>();
  a.token_s0 = tokens.stride(0);
  a.token_s1 = tokens.stride(1);
  a.accepted = accepted_len.data_ptr<int32_t>();
  a.accepted_s = accepted_len.stride(0);
  a.status = status.data_ptr<int32_t>();
  a.status_s = status.stride(0);
  a.path = path_used.data_ptr<int32_t>();
  a.path_s = path_used.stride(0);
  a.rows = rows;
  a.requests = requests;
  a.vocab = vocab;
  a.max_draft = max_draft;
  a.mode = int32_t(mode);
  a.dispatch = int32_t(dispatch);
  a.list_max = int32_t(list_max);
  a.workspace = workspace.data_ptr<uint8_t>();
  a.workspace_bytes = uint64_t(workspace.numel());

  c10::hip::HIPGuardMasqueradingAsCUDA guard(call.device());
  const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(call.device().index()).stream();
  const int32_t code = es_launch(&a, stream);
  if (code != ES_SUCCESS) {
    std::string detail = es_error_string(code);
    if (code == ES_ERR_LAUNCH) detail += std::string(" (") + es_last_hip_error() + ")";
    TORCH_CHECK(false, "exactsample kernel launch failed: ", detail);
  }
}
}  // namespace

TORCH_LIBRARY(exactsample, m) {
  m.def("verify_out(Tensor target_logits, Tensor cu_rows, Tensor draft_ids, Tensor? draft_logits, "
        "Tensor temperature, Tensor top_k, Tensor top_p, Tensor min_p, Tensor draft_kind, "
        "Tensor seeds, Tensor stream_ids, Tensor positions, Tensor? mask, "
        "Tensor(a!) workspace, Tensor(b!) tokens, Tensor(c!) accepted_len, Tensor(d!) status, "
        "Tensor(e!) path_used, int mode, int dispatch, int max_draft, int list_max) -> ()");
}
TORCH_LIBRARY_IMPL(exactsample, CUDA, m) { m.impl("verify_out", &verify_out); }
