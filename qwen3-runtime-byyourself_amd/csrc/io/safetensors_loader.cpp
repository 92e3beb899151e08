// SafetensorsLoader: one mapped file, its tensor table, and (for GPU
// batches) a staged upload kept across calls.  The behaviour callers see is
// that of the reference's src/io/safetensors_loader.cpp (results in request
// order, unknown names rejected before any transfer, every byte on the
// device when load_many returns); the transfer machinery is
// io_detail::StagedUpload.
#include "qwen3/io/safetensors_loader.h"

#include "staged_upload.hpp"

#include <stdexcept>

namespace qwen3
{
    SafetensorsLoader::SafetensorsLoader(const std::filesystem::path &model_path) : file_(model_path), metadata_(file_)
    {
    }

    SafetensorsLoader::~SafetensorsLoader() = default;

    Tensor SafetensorsLoader::load(std::string_view tensor_name, Device target_device) const
    {
        return io_detail::copy_out(file_, metadata_.tensor(tensor_name), target_device, tensor_name);
    }

    std::vector<Tensor> SafetensorsLoader::load_many(const std::vector<std::string> &tensor_names, Device target_device)
    {
        std::vector<Tensor> out;
        out.reserve(tensor_names.size());
        if (tensor_names.empty())
            return out;
        if (!target_device.is_cpu() && !target_device.is_cuda())
            throw std::invalid_argument("unsupported target device");
        std::vector<const SafetensorsTensorInfo *> infos;
        infos.reserve(tensor_names.size());
        std::size_t total = 0;
        for (const std::string &name : tensor_names)
        {
            infos.push_back(&metadata_.tensor(name));
            total += infos.back()->size_bytes();
        }
        if (target_device.is_cpu())
        {
            for (std::size_t i = 0; i < infos.size(); ++i)
                out.push_back(io_detail::copy_out(file_, *infos[i], target_device, tensor_names[i]));
            return out;
        }
        if (!upload_ || upload_->device() != target_device.index())
        {
            upload_.reset();
            upload_ = std::make_unique<io_detail::StagedUpload>(target_device.index());
        }
        const std::byte *data = file_.data_bytes().data();
        upload_->run(infos.size(), total, [&](std::size_t i) {
            const SafetensorsTensorInfo &info = *infos[i];
            out.push_back(Tensor::empty(info.shape, info.dtype, target_device));
            if (out.back().nbytes() != info.size_bytes())
                throw std::logic_error("Tensor size does not match metadata for '" + tensor_names[i] + "'");
            return io_detail::UploadPiece{data + info.begin_offset, out.back().data(), info.size_bytes()};
        });
        return out;
    }
} // namespace qwen3
