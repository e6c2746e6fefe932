# A dense layer's forward sums and adjoint scatters in STADE's generated form, with the weights
# row-major (k contiguous), an offset into x and index temporaries in the adjoint loop: a test
# text of the lowering's contractions (tests/test_lower_contract.py, tests/test_gpu_contract.py).
function dense_b(y, x, xb, w, wb, i_b, i_in, i_h)
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s = 0.5
        for i_k = 1:i_in
            s = s + w[(i_j - 1) * i_in + i_k] * x[(i_s - 1) * i_in + i_k + 2]
        end
        y[idx] = s
    end
    for idx = i_b * i_h:-1:1
        __t = idx - 1
        i_s = div(__t, i_h) + 1
        i_j = mod(__t, i_h) + 1
        sb = y[(i_s - 1) * i_h + i_j] * 2.0
        for i_k = i_in:-1:1
            __a = (i_j - 1) * i_in + i_k
            __c = (i_s - 1) * i_in + i_k + 2
            wb[__a] = wb[__a] + x[__c] * sb
            xb[__c] = xb[__c] + w[__a] * sb
        end
    end
    return nothing
end
