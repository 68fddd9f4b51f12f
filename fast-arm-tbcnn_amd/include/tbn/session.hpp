// tbn::InferenceSession (tbn-runtime/include/tbn/runtime/session.hpp:17-160).
// Same interface; one TBNModel::Session is kept for the lifetime of the
// InferenceSession, so weights are packed once (the reference builds a new
// Session, and repacks, on every run(), session.hpp:115).
#pragma once

#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "model.hpp"

namespace tbn {

// InferenceSession::Options (session.hpp:19-32).
struct InferenceSessionOptions {
    int num_threads = 1;               // accepted, unused (as in the reference)
    DeviceType device = DeviceType::HIP;
    bool enable_profiling = false;     // logs the wall time of run()
    bool enable_memory_pool = true;    // the device arena is always used
    size_t memory_pool_size = 16 * 1024 * 1024;
    bool use_quantization = false;
};

class InferenceSession {
public:
    using Options = InferenceSessionOptions;

    explicit InferenceSession(std::shared_ptr<TBNModel> model, const Options& options = Options());

    void initialize();
    void set_input(const std::string& name, const Tensor& tensor);
    Tensor get_input(const std::string& name) const;
    void run();
    Tensor get_output(const std::string& name) const;
    std::vector<std::string> get_input_names() const { return model_->inputs(); }
    std::vector<std::string> get_output_names() const { return model_->outputs(); }
    const Options& options() const { return options_; }
    double last_run_us() const { return last_run_us_; }

private:
    std::shared_ptr<TBNModel> model_;
    Options options_;
    bool initialized_ = false;
    std::unique_ptr<TBNModel::Session> session_;
    std::unordered_map<std::string, Tensor> inputs_;
    std::unordered_map<std::string, Tensor> outputs_;
    double last_run_us_ = 0.0;
};

std::unique_ptr<InferenceSession> create_inference_session(
    std::shared_ptr<TBNModel> model,
    const InferenceSession::Options& options = InferenceSession::Options());

}  // namespace tbn
